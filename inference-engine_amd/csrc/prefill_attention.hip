// Causal chunked-prefill attention over the int8 cache prefix (bf16 MFMA, gfx950).
#include "ie_common.h"

extern "C" hipError_t ie_prefill_attention(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, hipStream_t stream) {
    ie::set_error("prefill_attention: not built yet");
    return hipErrorNotSupported;
}
