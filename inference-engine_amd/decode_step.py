"""One greedy decode step of a Qwen3-1.7B-shaped model with the int8-KV attention path, captured
as a hipGraph: the harness for the whole-step measurement (tokens/s and the attention share).

Mirrors the decode branch of the reference's model (qwen3-1.7b/architecture.py:98-122 inside
TransformerBlock.forward :262-304 and Qwen3Model.forward :395-413) and its graph capture and
replay (qwen3-1.7b/engine.py:376-470): per layer, `add_rms_norm` (the first layer: RMSNorm),
QKV projection, `decode_attention_rope` (`fused_rope_kv_decode`'s norm + RoPE + int8 KV
write and `decode_attention` in one launch), output projection, `add_rms_norm`, gate/up
projection and `silu_mul` (one launch, `linear_silu_mul`, where the skinny GEMM serves that
shape), down projection; then the
final `add_rms_norm`, the tied-embedding LM head and greedy sampling (`sample` at tau 0,
kernels.py:1343-1370). All of these are this package's HIP kernels; for each projection
`linear` (kernels.py:1451-1458) runs this package's skinny GEMM or the library GEMM
(hipBLASLt), whichever `tune_linear` measured faster for that weight shape at the step's row
count before capture, as the reference's engine does (engine.py:352-374).

Fused form (`fused=True`, the default wherever the skinny GEMM serves all four layer
projections): both add_rms_norm launches of a layer go into the projections beside them. Each
RMSNorm weight is folded into the weight columns of the projection it feeds (input_norm into
qkv, post_norm into gate_up: `fold_rms_norm_weight`), which then normalizes the residual
stream's rows inside its own launch (`linear_norm`), and o_proj and down add their output to the
residual stream in place (`linear_residual_`, bit for bit add_rms_norm's new residual). Per
layer five launches instead of seven; the normalized rows differ from the two-launch form only
in where the bf16 rounding falls (the folded weight is rounded instead of the normalized row).

Weights are random (bf16, std 0.02) and the caches hold random int8 K/V: there is no checkpoint
here, and the step's cost does not depend on the values.
"""

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch.cuda import nvtx

from .attention_layer import attention, rope_inv_freq, rope_tables
from .kernels import (LayerKVCache, add_rms_norm, decode_attention_rope, decode_plan,
                      decode_step_prologue,
                      fold_rms_norm_weight, linear, linear_norm, linear_residual_,
                      linear_silu_mul, lm_head_greedy, make_layer_cache, sample, skinny_matmul,
                      swizzle_weight,
                      swizzled_tiles, tune_linear, use_skinny, use_skinny_glu)


@dataclass(frozen=True)
class Qwen3Shape:
    """qwen3-1.7b/architecture.py:492-500."""

    model_dim: int = 2048
    intermediate: int = 6144
    head_dim: int = 128
    num_q_heads: int = 16
    num_kv_heads: int = 8
    vocab: int = 151936
    layers: int = 28
    rope_base: float = 1e6
    eps: float = 1e-6


@dataclass
class LayerWeights:
    input_norm: torch.Tensor  # [model_dim]
    qkv: torch.Tensor  # [(Hq + 2 Hkv) D, model_dim]
    q_norm: torch.Tensor  # [D]
    k_norm: torch.Tensor  # [D]
    o_proj: torch.Tensor  # [model_dim, Hq D]
    post_norm: torch.Tensor  # [model_dim]
    gate_up: torch.Tensor  # [2 intermediate, model_dim]
    down: torch.Tensor  # [model_dim, intermediate]


def random_weights(shape: Qwen3Shape, device, seed=0, std=0.02):
    g = torch.Generator(device=device).manual_seed(seed)

    def w(*dims):
        return (torch.randn(*dims, generator=g, device=device, dtype=torch.float32) * std).bfloat16()

    def ones(n):
        return torch.ones(n, device=device, dtype=torch.bfloat16)

    D, H = shape.head_dim, shape.model_dim
    layers = [
        LayerWeights(
            input_norm=ones(H),
            qkv=w((shape.num_q_heads + 2 * shape.num_kv_heads) * D, H),
            q_norm=ones(D),
            k_norm=ones(D),
            o_proj=w(H, shape.num_q_heads * D),
            post_norm=ones(H),
            gate_up=w(2 * shape.intermediate, H),
            down=w(H, shape.intermediate),
        )
        for _ in range(shape.layers)
    ]
    embed = w(shape.vocab, H)
    return layers, embed, ones(H)


def random_caches(shape: Qwen3Shape, pool: int, max_len: int, device, seed=0):
    """Per-layer int8 caches with random content in every column (scales ~0.02)."""
    g = torch.Generator(device=device).manual_seed(seed + 1)
    caches = []
    for _ in range(shape.layers):
        c = make_layer_cache(pool, shape.num_kv_heads, max_len, shape.head_dim, device=device)
        c.k.copy_(torch.randint(-127, 128, c.k.shape, generator=g, device=device, dtype=torch.int8))
        c.v.copy_(torch.randint(-127, 128, c.v.shape, generator=g, device=device, dtype=torch.int8))
        c.k_scale.copy_(torch.rand(c.k_scale.shape, generator=g, device=device) * 0.04)
        c.v_scale.copy_(torch.rand(c.v_scale.shape, generator=g, device=device) * 0.04)
        caches.append(c)
    return caches


class DecodeStep:
    """Static-address decode step for B sequences (engine.py:376-412): the graph reads ids,
    cached_lens and slot_ids from fixed tensors, which the caller rewrites between replays."""

    def __init__(self, shape: Qwen3Shape, layers, embed, final_norm, caches: list[LayerKVCache],
                 batch: int, device, fused: bool = False, swizzle: bool | None = None):
        """fused: fold every layer's input_norm into its qkv weight and post_norm into its
        gate_up weight, in place (the layers then serve only the fused form). swizzle (default:
        with fused): every projection weight for which tune_linear timed the skinny GEMM faster
        on the weight in the GEMM's fragment order (swizzled_tiles: the tile width) is reordered
        in place into that order for that width (swizzle_weight; the row-major weight's result
        bits at that width); the LM head gets a reordered copy of the embedding."""
        self.shape, self.layers, self.embed, self.final_norm = shape, layers, embed, final_norm
        self.fused = fused
        self.swz = dict.fromkeys(("qkv", "o_proj", "gate_up", "down", "lm_head"), False)
        self.swz_tiles = dict.fromkeys(self.swz)
        self.lm_head_w = embed
        if fused:
            for lw in layers:
                lw.qkv = fold_rms_norm_weight(lw.qkv, lw.input_norm)
                lw.gate_up = fold_rms_norm_weight(lw.gate_up, lw.post_norm)
            self._zero = torch.zeros(batch, shape.model_dim, device=device, dtype=torch.bfloat16)
            if swizzle is None or swizzle:
                lw = layers[0]
                tiles = lambda w, glu=False: swizzled_tiles(w.shape[0], w.shape[1], batch, glu)
                nt = {name: tiles(getattr(lw, name)) for name in ("qkv", "o_proj", "down")}
                nt["gate_up"] = tiles(lw.gate_up, True)
                nt["lm_head"] = tiles(embed)
                self.swz_tiles = nt
                for name, t in nt.items():
                    self.swz[name] = t is not None
                for lw in layers:
                    for name in ("qkv", "o_proj", "gate_up", "down"):
                        if self.swz[name]:
                            setattr(lw, name, swizzle_weight(getattr(lw, name), nt[name],
                                                             gate_up=name == "gate_up"))
                if self.swz["lm_head"]:  # the final RMSNorm's weight folded in as well
                    self.lm_head_w = swizzle_weight(fold_rms_norm_weight(embed, final_norm),
                                                    nt["lm_head"])
        self.caches = caches
        self.B = batch
        pool = caches[0].k.shape[0]
        assert batch <= pool
        self.ids = torch.zeros(batch, device=device, dtype=torch.int64)
        self.cached_lens = torch.zeros(batch, device=device, dtype=torch.int32)
        self.slot_ids = torch.arange(batch, device=device, dtype=torch.int32)
        self.num_decoding = torch.full((1,), batch, device=device, dtype=torch.int32)
        self.seed = torch.zeros(1, device=device, dtype=torch.int64)  # the engine's sampling seed
        self.inv_freq = rope_inv_freq(shape.head_dim, shape.rope_base, device)
        self.graph = None
        self.graph_out = None

    def _rope(self):
        # decode: a token's position is the number of tokens before it (architecture.py:382-390)
        return rope_tables(self.cached_lens, self.inv_freq)

    def _rms(self, x, w):
        return F.rms_norm(x.float(), (x.shape[-1],), w.float(), self.shape.eps).bfloat16()

    def attention(self, li, normed, cos, sin):
        """AttentionLayer.forward, pure-decode branch (architecture.py:85-122), through
        attention_layer.attention."""
        lw, B = self.layers[li], self.B
        assert not self.fused
        with nvtx.range("qkv_proj"):
            qkv = linear(normed, lw.qkv)
        out = self._attend(li, qkv, cos, sin)
        with nvtx.range("o_proj"):
            return linear(out.view(B, -1), lw.o_proj)

    def _attend(self, li, qkv, cos, sin, plan=None):
        s, lw, B = self.shape, self.layers[li], self.B
        q, k, v = qkv.split([s.num_q_heads * s.head_dim, s.num_kv_heads * s.head_dim,
                             s.num_kv_heads * s.head_dim], dim=-1)
        q = q.view(B, s.num_q_heads, s.head_dim)
        k = k.view(B, s.num_kv_heads, s.head_dim)
        v = v.view(B, s.num_kv_heads, s.head_dim)
        return attention(q, k, v, None, None, cos, sin, self.caches[li], self.cached_lens,
                         self.slot_ids, None, 0, None, self.num_decoding, lw.q_norm, lw.k_norm,
                         s.eps, decode_plan=plan)

    def forward(self) -> torch.Tensor:
        """One step: returns the greedy next token of every sequence, int64 [B, 1]."""
        if self.swz["lm_head"] and self.embed.shape[1] == 2048:
            # LM head (final RMSNorm inside) and greedy sampling in one launch
            h = self.hidden(final_norm=False)
            with nvtx.range("lm_head+sample"):
                return lm_head_greedy(h, self.lm_head_w, self.seed, self.shape.eps)[1]
        logits = self.logits()
        with nvtx.range("sample"):
            return sample(logits, 0.0, self.seed)

    def logits(self) -> torch.Tensor:
        """The step up to the LM head: bf16 [B, vocab]. With a reordered LM head weight (the
        fused form) the final RMSNorm runs inside the LM head's launch, its weight folded into
        that copy of the embedding."""
        fold = self.swz["lm_head"]
        h = self.hidden(final_norm=not fold)
        with nvtx.range("lm_head"):
            if fold:  # the residual stream's RMSNorm inside the GEMM (IE_SKINNY_NORM)
                return linear_norm(h, self.lm_head_w, self.shape.eps, swizzled=True)
            return linear(h, self.embed)

    def hidden(self, final_norm: bool = True) -> torch.Tensor:
        """The step up to the final RMSNorm: bf16 [B, model_dim], the LM head's input
        (final_norm=False, fused form: the residual stream before that norm)."""
        # the reference's ranges (architecture.py:278-304, 379-413, 477; engine.py:216)
        if self.fused:  # embedding rows, RoPE tables and the decode work list: one launch
            s = self.shape
            with nvtx.range("embed+metadata"):
                x, plan, cos, sin = decode_step_prologue(
                    self.ids, self.embed, self.cached_lens, self.num_decoding, s.num_q_heads,
                    s.num_kv_heads, self.inv_freq)
            return self._hidden_fused(x, cos, sin, plan, final_norm)
        with nvtx.range("embed"):
            x = F.embedding(self.ids, self.embed)
        with nvtx.range("metadata"):
            cos, sin = self._rope()
        residual = None
        eps = self.shape.eps
        for li, lw in enumerate(self.layers):
            with nvtx.range("layer"):
                with nvtx.range("attn"):
                    if residual is None:  # architecture.py:280-281: the first block norms its input
                        residual, normed = x, self._rms(x, lw.input_norm)
                    else:
                        residual, normed = add_rms_norm(residual, x, lw.input_norm, eps)
                    attn = self.attention(li, normed, cos, sin)
                with nvtx.range("mlp"):
                    residual, normed = add_rms_norm(residual, attn, lw.post_norm, eps)
                    x = linear(linear_silu_mul(normed, lw.gate_up), lw.down)
        with nvtx.range("final_norm"):
            _, h = add_rms_norm(residual, x, self.final_norm, eps)
        return h

    def _hidden_fused(self, x, cos, sin, plan, final_norm=True):
        """The layers in the fused form: h, the residual stream, is the embedding's output
        (a new tensor every step), updated in place by o_proj and down; plan, the decode
        launch's work list, serves every layer."""
        eps, h, sw = self.shape.eps, x, self.swz
        for li, lw in enumerate(self.layers):
            with nvtx.range("layer"):
                with nvtx.range("attn"):
                    with nvtx.range("qkv_proj"):  # input_norm inside (folded into lw.qkv)
                        qkv = linear_norm(h, lw.qkv, eps, swizzled=sw["qkv"])
                    out = self._attend(li, qkv, cos, sin, plan)
                    with nvtx.range("o_proj"):  # + the residual add of the post-norm
                        linear_residual_(out.view(self.B, -1), lw.o_proj, h,
                                         swizzled=sw["o_proj"])
                with nvtx.range("mlp"):  # post_norm inside (folded into lw.gate_up)
                    # a paired gate/up weight writes the activation in the fragment order the
                    # down projection reads without an LDS round trip
                    frag = sw["gate_up"]
                    act = linear_norm(h, lw.gate_up, eps, silu_mul=True, swizzled=frag,
                                      fragments=frag)
                    linear_residual_(act, lw.down, h, swizzled=sw["down"], x_fragments=frag)
        if not final_norm:
            return h
        with nvtx.range("final_norm"):  # h already holds the last down projection's sum
            _, hn = add_rms_norm(h, self._zero, self.final_norm, eps)
        return hn

    def attention_only(self) -> torch.Tensor:
        """The step's attention kernels alone (per layer: decode_attention_rope, i.e.
        fused_rope_kv_decode and decode_attention in one launch, on fixed activations; in the
        fused form with the step's decode work list, as the step runs them), for the attention
        share of a step."""
        s, B = self.shape, self.B
        cos, sin = self._rope()
        if not hasattr(self, "_qkv_fixed"):
            g = torch.Generator(device=self.ids.device).manual_seed(7)
            self._qkv_fixed = torch.randn(B, (s.num_q_heads + 2 * s.num_kv_heads) * s.head_dim,
                                          generator=g, device=self.ids.device).bfloat16()
        q, k, v = self._qkv_fixed.split([s.num_q_heads * s.head_dim, s.num_kv_heads * s.head_dim,
                                         s.num_kv_heads * s.head_dim], dim=-1)
        q = q.view(B, s.num_q_heads, s.head_dim)
        k = k.view(B, s.num_kv_heads, s.head_dim)
        v = v.view(B, s.num_kv_heads, s.head_dim)
        out = None
        plan = decode_plan(self.cached_lens, self.num_decoding, B, s.num_q_heads,
                           s.num_kv_heads) if self.fused else None
        for li, lw in enumerate(self.layers):
            out = decode_attention_rope(q, k, v, lw.q_norm, lw.k_norm, cos, sin, self.slot_ids,
                                        self.caches[li], self.cached_lens, self.num_decoding,
                                        s.eps, s.head_dim ** -0.5, plan=plan)
        return out

    def capture(self, fn=None):
        """Warm up twice on a side stream, then capture `fn` (default: forward) into a hipGraph
        (engine.py:432-449). Returns (graph, output tensor the replays overwrite)."""
        fn = fn or self.forward
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):  # the warmed-up stream: its workspaces exist
            out = fn()
        return graph, out


def make_decode_step(batch=32, ctx_lo=128, ctx_hi=4096, shape=Qwen3Shape(), device="cuda",
                     seed=0, tune=True, fused=None, norm_std=0.0, swizzle=None):
    """Config-5 step: B sequences with cached lengths ~ U[ctx_lo, ctx_hi) - 1 (the new token is
    the ctx-th), slots 0..B-1 of a pool of B + 1 (the last row is the engine's scratch slot).
    fused=None: the fused form wherever tune_linear chose the skinny GEMM for all four layer
    projections at this batch (always the case at B = 32). norm_std > 0: RMSNorm weights
    1 + norm_std * N(0, 1) instead of ones."""
    layers, embed, final_norm = random_weights(shape, device, seed)
    if norm_std > 0:
        g = torch.Generator(device=device).manual_seed(seed + 2)
        for t in [final_norm] + [n for lw in layers for n in (lw.input_norm, lw.post_norm)]:
            t.copy_(1 + norm_std * torch.randn(t.shape, generator=g, device=device))
    caches = random_caches(shape, batch + 1, ctx_hi, device, seed)
    if tune:  # one weight of every shape (the table is keyed by shape)
        lw = layers[0]
        tune_linear([lw.qkv, lw.o_proj, lw.gate_up, lw.down, embed], [batch])
    if fused is None:
        lw = layers[0]
        fused = all(use_skinny.get((w.shape[0], w.shape[1], batch)) is not None
                    for w in (lw.qkv, lw.o_proj, lw.gate_up, lw.down)) and \
            (lw.gate_up.shape[0], lw.gate_up.shape[1], batch) in use_skinny_glu
    step = DecodeStep(shape, layers, embed, final_norm, caches, batch, device, fused=fused,
                      swizzle=swizzle)
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi, (batch,), generator=g)
    step.cached_lens.copy_((ctx - 1).to(torch.int32))
    step.ids.copy_(torch.randint(0, shape.vocab, (batch,), generator=g))
    return step


def _main():
    """Replay the config-5 step graph (for kernel traces): python -m <package>.decode_step"""
    import argparse

    ap = argparse.ArgumentParser()
    ap.add_argument("--replays", type=int, default=20)
    ap.add_argument("--attention-only", action="store_true")
    ap.add_argument("--eager", type=int, default=0, metavar="N",
                    help="run N steps without a graph instead (their NVTX/roctx stage ranges "
                         "are then recorded at every step, for a marker trace)")
    args = ap.parse_args()
    step = make_decode_step(device="cuda:0")
    if args.eager:
        for _ in range(args.eager):
            out = step.forward()
        torch.cuda.synchronize()
        print(f"ran {args.eager} eager steps; first tokens {out.view(-1)[:4].tolist()}",
              flush=True)
        return
    graph, out = step.capture(step.attention_only if args.attention_only else None)
    for _ in range(args.replays):
        graph.replay()
    torch.cuda.synchronize()
    print(f"replayed {args.replays} steps; first tokens {out.view(-1)[:4].tolist()}; "
          f"tuned skinny tile widths: row-major {use_skinny}, gate/up {use_skinny_glu}, "
          f"reordered weights {step.swz_tiles}", flush=True)


if __name__ == "__main__":
    _main()
