"""CPU oracle for the int8-KV attention path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, in numpy, the arithmetic of kbwal/inference-engine's attention kernels
(qwen3-1.7b/kernels.py) so the HIP path can be checked against it. Only tests/, the
`smoke()` function of __graft_entry__.py and the `cpu_baseline` leg of bench.py may import it,
and only as the checker: the product package never imports, links or runs anything here.

Modules
  numerics   bf16 rounding, the fixed-order wave butterfly sum
  kv_cache   quantize-on-write (prefill and decode), prefix dequantize, cache containers,
             the prefill q/k RMSNorm + RoPE
  sampling   Gumbel-max token sampling with Triton's Philox4x32-10 uniforms (greedy at tau 0)
  attention  decode attention (reference rounding points, split-K form, float64 textbook)
             and causal chunked-prefill attention
  work_split the split-K work partition of the decode kernel (integer restatement)
  torch_cpu  the same decode / KV write / prefill math in PyTorch fp32 on the host cores: the
             benchmark's CPU baseline (bench.py's cpu_baseline leg only)

Pinning (what checks each function independently of this restatement; see tests/test_oracle_*):
  quantize_rows / calibration   closed-form known answers (zero rows, one-hot, exact ties, clamp,
                                calibration floor), brute-force round-trip bound |x - q*s| <= s/2
  fused_rope_kv_decode          RMSNorm against torch.nn.RMSNorm in float64, RoPE against complex
                                multiplication in float64, quantize pinned as above
  fused_norm_rope_prefill       the same float64 forms, known answers (constant rows, zero and
                                quarter-turn angles), equality with the decode rotation
  sampling                      Philox4x32-10 against the Random123 known-answer vectors, the
                                uniform map's closed forms, greedy = first argmax, tau > 0
                                frequencies against softmax(logits / tau)
  dequantize_kv_prefix          closed form on hand-built int8 rows
  decode_attention              float64 torch scaled_dot_product_attention on the dequantized
                                cache; split-K merge equal to the unsplit form
  prefill_attention             float64 torch scaled_dot_product_attention with an explicit
                                causal+prefix mask; brute-force per-row loop on tiny shapes
  decode_work_plan              brute-force coverage properties (every token of every decoding
                                sequence covered exactly once, <= target+B work items)
  torch_cpu                     decode and prefill against the float64 textbook forms (2e-5),
                                the KV write bit for bit against quantize_kv_prefill
The reference ships no tests, golden vectors or fixtures (it has no test suite at all), so no
reference-held vector pins any function; the reference kernels need a GPU and Triton and are not
run here.
"""
