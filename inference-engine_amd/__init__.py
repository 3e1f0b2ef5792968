"""MI355X-native int8-KV attention path of kbwal/inference-engine.

Drop-in for the reference's attention kernel API (qwen3-1.7b/kernels.py): int8 quantize-on-write,
split-K GQA decode attention, causal chunked-prefill attention on bf16 MFMA, the prefill q/k
RMSNorm + RoPE, token sampling, the per-layer add_rms_norm / silu_mul, and hipGraph capture of
the decode step. The directory name is not a Python identifier, so import it with
`importlib.import_module("inference-engine_amd")`.
"""

from . import attention_layer, kernels, step_inputs  # noqa: F401
from .kernels import (  # noqa: F401
    LayerKVCache,
    add_rms_norm,
    decode_attention,
    decode_attention_rope,
    decode_plan,
    decode_step_prologue,
    dequantize_kv_prefix,
    fold_rms_norm_weight,
    fused_norm_rope_prefill,
    fused_rope_kv_decode,
    make_layer_cache,
    prefill_attention,
    prefill_plan,
    quantize_kv_prefill,
    sample,
    silu_mul,
    skinny_matmul,
    skinny_matmul_silu_mul,
    swizzle_weight,
    linear,
    linear_norm,
    linear_residual_,
    linear_silu_mul,
    lm_head_greedy,
    tune_linear,
)
