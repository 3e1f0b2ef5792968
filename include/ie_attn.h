/*
 * ie_attn.h — C ABI of the MI355X (gfx950) int8-KV attention path.
 *
 * One shared library, libie_attn.so, exports these entry points. Every pointer is a device
 * pointer, every stride is in elements (not bytes), every call is asynchronous on `stream`,
 * allocates nothing, never synchronises, and reads per-step counts (`num_decoding`,
 * `cached_lens`, `cu_seqlens`, ...) on the device only, so every call can be captured into a
 * hipGraph. Grids depend on shapes alone.
 *
 * Geometry supported by the attention and KV-cache kernels: head_dim 128 and 1 to 16 query
 * heads per KV head (Qwen3-1.7B: 16 query heads over 8 KV heads, ratio 2, the tuned case).
 * Other geometries return hipErrorInvalidValue.
 *
 * Each entry point replaces one Python wrapper of kbwal/inference-engine's Triton kernel API,
 * cited as qwen3-1.7b/kernels.py:<line>, with the same argument meaning. Bit-level contracts:
 *   - int8 values and fp32 scales written by the two quantizing entry points are computed with
 *     IEEE round-to-nearest-even fp32 operations in a fixed order (documented per function),
 *   - attention outputs are bf16, rounded to nearest even from fp32 accumulators.
 */
#ifndef IE_ATTN_H
#define IE_ATTN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 values travel as their 16-bit patterns. */
typedef uint16_t ie_bf16;

/* Element types an entry point may take at run time. */
enum { IE_DTYPE_BF16 = 0, IE_DTYPE_F32 = 1 };

/*
 * One layer's int8 KV cache (qwen3-1.7b/kernels.py:11-17 `LayerKVCache`; allocated by
 * qwen3-1.7b/engine.py:472-492). Layout, unchanged from the reference:
 *   k, v           int8  [pool, num_kv_heads, max_len, head_dim]
 *   k_scale,v_scale fp32 [pool, num_kv_heads, max_len]
 *   k_calibration  fp32  [pool, num_kv_heads, 1, head_dim]
 * k and v share one set of strides, k_scale and v_scale share another
 * (the reference asserts both, kernels.py:284-287). head_dim and the token axis of the scales
 * must be unit-stride.
 */
typedef struct ie_kv_cache {
    int8_t* k;
    int8_t* v;
    float* k_scale;
    float* v_scale;
    float* k_calibration;
    int64_t pool;
    int64_t num_kv_heads;
    int64_t max_len;
    int64_t head_dim;
    int64_t stride_slot;       /* k/v stride of dim 0 */
    int64_t stride_head;       /* k/v stride of dim 1 */
    int64_t stride_tok;        /* k/v stride of dim 2 */
    int64_t scale_stride_slot; /* k_scale/v_scale stride of dim 0 */
    int64_t scale_stride_head; /* k_scale/v_scale stride of dim 1 */
    int64_t cal_stride_slot;   /* k_calibration stride of dim 0 */
    int64_t cal_stride_head;   /* k_calibration stride of dim 1 */
} ie_kv_cache;

/* Library version, (major << 16) | minor. */
int32_t ie_attn_version(void);

/* Human-readable name of the last argument error seen on this thread, or "" if none. */
const char* ie_attn_last_error(void);

/*
 * Measurement helper, no counterpart in the reference: reads `bytes` (a multiple of 16, 16-byte
 * aligned) from device memory p once, at the device's attainable rate (8 workgroups of 256
 * per CU, each streaming a contiguous 1/G of the buffer with 16-byte loads, eight in flight).
 * Each thread XORs the 32-bit words it read and writes that value to out[0] only if it equals
 * `never`. Used to put the decode kernel's HBM rate beside what a pure read stream reaches on
 * the same device.
 */
hipError_t ie_hbm_read_probe(const void* p, size_t bytes, uint32_t never, uint32_t* out,
                             hipStream_t stream);

/*
 * Quantize-on-write for prefilling entries.
 * Replaces qwen3-1.7b/kernels.py:826-865 `quantize_kv_prefill(k, v, cu_seqlens, slot_ids,
 * cached_lens, num_decoding, cache)` (kernel kernels.py:717-823).
 *
 * k, v: bf16 [N, num_kv_heads, head_dim], any token/head strides (v is usually a strided view of
 * the fused qkv output). Entry b (num_decoding[0] <= b < num_entries, chunk_len > 0) writes its
 * packed tokens [cu_seqlens[b], cu_seqlens[b+1]) to cache row slot_ids[b] starting at column
 * cached_lens[b]. When cached_lens[b] == 0 the per-channel K calibration of that row is first
 * recomputed as max(1e-3, max_t |k[t, d]|) over the chunk and stored; otherwise it is read.
 * Per token and head: x = k / cal; s = max(max|x|, 1e-6) / 127; q = clamp(rint(x / s), ±127).
 * V uses the same formula with cal = 1.
 * One launch when num_tokens <= 1536 (each workgroup derives the calibration itself); two
 * launches otherwise (the per-channel max of every first chunk, then a streaming quantize
 * launch), so the cost stays linear in the chunk length. Both forms write identical bytes.
 * cdiv(num_tokens, 32) + num_entries must not exceed 65535 (about two million tokens per step).
 */
hipError_t ie_quantize_kv_prefill(const ie_bf16* k, int64_t k_stride_tok, int64_t k_stride_head,
                                  const ie_bf16* v, int64_t v_stride_tok, int64_t v_stride_head,
                                  int64_t num_tokens,
                                  const int32_t* cu_seqlens, const int32_t* slot_ids,
                                  const int32_t* cached_lens, const int32_t* num_decoding,
                                  int32_t num_entries, const ie_kv_cache* cache,
                                  hipStream_t stream);

/*
 * Decode-side q/k RMSNorm + RoPE + calibration fold + K/V quantize-on-write.
 * Replaces qwen3-1.7b/kernels.py:483-544 `fused_rope_kv_decode(q, k, v, q_norm_weight,
 * k_norm_weight, cos, sin, slot_ids, kv_cache, cached_lens, num_decoding, eps)`
 * (kernel kernels.py:364-480).
 *
 * q: bf16 [B, num_q_heads, head_dim]; k, v: bf16 [B, num_kv_heads, head_dim] (strided views
 * allowed); q_norm_weight, k_norm_weight: bf16 [head_dim]; cos, sin: bf16 [B, 1, head_dim/2].
 * For b < num_decoding[0]: q_out[b, h] = bf16(rope(rmsnorm(q[b, h])) * cal[slot, h / 2]) and the
 * int8 K (rope(rmsnorm(k)) / cal) and V with their scales are written at column cached_lens[b]
 * of row slot_ids[b]. Rows b >= num_decoding[0] of q_out are left untouched.
 * RMSNorm: sum of squares of each 64-element half by a butterfly over lane distance
 * 32,16,8,4,2,1, halves added, / head_dim, + eps, rstd = 1 / sqrt(.) (both IEEE).
 */
hipError_t ie_fused_rope_kv_decode(const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const ie_bf16* k, int64_t k_stride_b, int64_t k_stride_h,
                                   const ie_bf16* v, int64_t v_stride_b, int64_t v_stride_h,
                                   const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
                                   const ie_bf16* cos, int64_t cos_stride_b,
                                   const ie_bf16* sin, int64_t sin_stride_b,
                                   const int32_t* slot_ids, const int32_t* cached_lens,
                                   const int32_t* num_decoding, int32_t batch,
                                   int32_t num_q_heads, float eps, const ie_kv_cache* cache,
                                   ie_bf16* q_out, int64_t q_out_stride_b,
                                   int64_t q_out_stride_h, hipStream_t stream);

/*
 * Bytes of device workspace ie_decode_attention needs for `batch` sequences of num_q_heads query
 * heads on the current device, whatever the GQA ratio: the arrival counts (one uint32 per
 * sequence and query head, the most any ratio uses, with room for max(batch, 1024) sequences of
 * max(num_q_heads, 128) heads, padded to 256 bytes), then fp32 split-K partials, head_dim + 2
 * values per (query head, work entry), where the work entries are at most
 * ie_decode_attention_grid(batch, cdiv(num_q_heads, 2)). The arrival counts must be zero when a
 * workspace is first used (allocate it zeroed); every call that completes leaves them zero
 * again, so one workspace (of the largest size any of them needs) serves any number of calls in
 * stream order of any batch up to 1024 and any num_q_heads up to 128 (they share one count
 * region). A workspace used with a larger batch or head count serves that shape only, unless
 * zeroed again.
 */
size_t ie_decode_attention_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim);

/*
 * The leading bytes of a decode workspace for `batch` sequences that must be zero on entry (the
 * arrival counts: max(batch, 1024) * num_kv_heads uint32, padded to 256 bytes). Zeroing them
 * resets a workspace, e.g. one whose memory was reused or a launch that did not complete, and
 * a caller that records the decode call into a hipGraph from freshly allocated memory records
 * a fill of these bytes first. (max(batch, 1024) * num_q_heads uint32, padded to 256 bytes.) No counterpart in the reference (its partials need no counts).
 */
size_t ie_decode_attention_workspace_counts_bytes(int32_t batch, int32_t num_q_heads);

/* Upper bound on splits per sequence on the current device: the largest per-unit workgroup
 * target of any launch shape (CUs * 8 / num_units, 2-wave workgroups). A unit is a KV head and
 * one pair of its query heads: num_units = num_kv_heads * cdiv(num_q_heads / num_kv_heads, 2),
 * num_kv_heads itself at GQA ratio 2. */
int32_t ie_decode_attention_max_splits(int32_t num_units);

/*
 * The per-unit workgroup target of the work split (qwen3-1.7b/kernels.py:20-37 TARGET) that
 * ie_decode_attention uses for `batch` sequences on the current device (num_units as above). The
 * launch fills the CUs with 16 waves each, as 8-wave workgroups (target CUs * 2 / num_units)
 * while the batch fits that target, else as 4-wave (CUs * 4 / num_units) or 2-wave (CUs * 8 /
 * num_units) workgroups, the first whose target holds the batch (the 2-wave one above that).
 */
int32_t ie_decode_attention_target(int32_t batch, int32_t num_units);

/*
 * Split-K GQA decode attention over the int8 cache, with the partial-softmax reduce folded into
 * the same launch (the sequence's last piece to finish merges its pieces). Any GQA ratio
 * num_q_heads / num_kv_heads of 1 to 16 (the reference's q-group padding, kernels.py:118-135),
 * head_dim 128; a workgroup serves one pair of a KV head's query heads, so ratios above 2 read
 * each KV row once per pair.
 * Replaces qwen3-1.7b/kernels.py:272-361 `decode_attention(q, kv_cache, cached_lens, slot_ids,
 * num_decoding, scale, out)` (kernels kernels.py:73-213 and 216-264, work split 20-70).
 *
 * q: bf16 [B, num_q_heads, head_dim], calibration already folded in. Sequence b < num_decoding[0]
 * attends to tokens [0, cached_lens[b] + 1) of cache row slot_ids[b]:
 *   out[b, h] = sum_t softmax_t(scale * k_scale[t] * <q[b, h], k[t]>) * v_scale[t] * v[t].
 * Only rows b < num_decoding[0] of out are written. `workspace` must hold
 * ie_decode_attention_workspace_size(B, num_q_heads, head_dim) bytes with its arrival counts
 * zero (see there); calls that share a workspace must not overlap.
 */
hipError_t ie_decode_attention(const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h,
                               int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
                               const int32_t* cached_lens, const int32_t* slot_ids,
                               const int32_t* num_decoding, float scale, ie_bf16* out,
                               int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/*
 * ie_fused_rope_kv_decode followed by ie_decode_attention, in one launch: the decode branch of
 * the attention layer (qwen3-1.7b/architecture.py:113-122, which calls kernels.py:483-544 and
 * then kernels.py:272-361). No single counterpart in the reference: the two reference calls it
 * replaces stay available as the two entry points above.
 *
 * q: bf16 [B, num_q_heads, head_dim], the QKV projection's raw rows (before norm and RoPE; any
 * strides with unit channel stride); k, v, q_norm_weight, k_norm_weight, cos, sin, eps as for
 * ie_fused_rope_kv_decode; the remaining arguments as for ie_decode_attention (same workspace).
 * For every sequence b < num_decoding[0]: the cache afterwards holds the bits
 * ie_fused_rope_kv_decode writes (int8 K and V and their scales at column cached_lens[b] of row
 * slot_ids[b]), and out[b] is decode attention with the q that ie_fused_rope_kv_decode would
 * return (its bits); q_out itself is not produced. Within the launch the piece of each sequence
 * that ends at the new token computes that token's K/V row, writes it to the cache and uses its
 * own copy (in LDS); no piece reads that column from the cache.
 */
hipError_t ie_decode_attention_rope(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    float eps, int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
    const int32_t* cached_lens, const int32_t* slot_ids, const int32_t* num_decoding,
    float scale, ie_bf16* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, hipStream_t stream);

/*
 * ie_decode_attention without a workspace argument, for callers that cannot allocate device
 * memory (code under hipGraph capture, serving loops and harnesses that forbid allocation). No
 * counterpart in the reference. The arrival counts and split-K partials live in a static device
 * array of ie_decode_attention_noalloc_max_bytes() bytes (16 MiB) that each device the library
 * runs on holds until the process ends; a batch above 1024 sequences returns
 * hipErrorInvalidValue. Allocates
 * nothing; the first call on a device looks up the array's address there (make it outside
 * graph capture). Every call on a device shares the array: calls that overlap on one device
 * race. Same arguments, results and errors as ie_decode_attention otherwise.
 */
size_t ie_decode_attention_noalloc_max_bytes(void);
hipError_t ie_decode_attention_noalloc(const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h,
                                       int32_t batch, int32_t num_q_heads,
                                       const ie_kv_cache* cache, const int32_t* cached_lens,
                                       const int32_t* slot_ids, const int32_t* num_decoding,
                                       float scale, ie_bf16* out, int64_t out_stride_b,
                                       int64_t out_stride_h, hipStream_t stream);

/*
 * The decode launch's work list, for tests and diagnostics: the work split of
 * qwen3-1.7b/kernels.py:20-70 (`compute_piece`, `assign_work`) as the decode kernel computes it
 * on the device. ie_decode_attention_grid(batch, num_units) is the number of work entries
 * (the decode launch's workgroups per unit: KV head x query-head pair, as above); ie_decode_attention_plan writes, for each entry
 * w, rows[4w .. 4w+3] = (sequence b, split index, splits of b, piece size in tokens), with
 * splits = 0 for an entry that has no work. rows: int32 [grid, 4] device memory.
 */
int32_t ie_decode_attention_grid(int32_t batch, int32_t num_units);
hipError_t ie_decode_attention_plan(const int32_t* cached_lens, const int32_t* num_decoding,
                                    int32_t batch, int32_t num_units, int32_t* rows,
                                    hipStream_t stream);

/*
 * A decode step's per-step inputs in one launch (no counterpart in the reference, which runs
 * the embedding lookup, the RoPE table arithmetic and the attention metadata as separate
 * kernels, architecture.py:379-413 / engine.py:216): the work list of ie_decode_attention_plan
 * (rows, as that call writes them), the RoPE tables of ie_rope_tables for positions
 * cached_lens[0 .. batch) (cos_out / sin_out: bf16 [batch, half_dim]), and the embedding rows
 * x[b, :] = embed[ids[b], :] (bf16, model_dim a multiple of 8, 16-byte aligned rows; an id
 * outside [0, vocab) gives a zero row). The same bits as the three separate calls.
 */
hipError_t ie_decode_step_prologue(const int32_t* cached_lens, const int32_t* num_decoding,
                                   int32_t batch, int32_t num_units, int32_t* rows,
                                   const float* inv_freq, int32_t half_dim, ie_bf16* cos_out,
                                   ie_bf16* sin_out, const int64_t* ids, const ie_bf16* embed,
                                   int64_t embed_stride, int64_t vocab, int32_t model_dim,
                                   ie_bf16* x, int64_t x_stride, hipStream_t stream);

/*
 * ie_decode_attention and ie_decode_attention_rope with their work list precomputed (no
 * counterpart in the reference): the same arguments and results, plus `plan`, the rows
 * ie_decode_attention_plan wrote for the same cached_lens and num_decoding values, batch,
 * num_units (KV heads x query-head pairs) and device, 16-byte aligned, and plan_rows, their
 * count (at least ie_decode_attention_grid(batch, num_units)). Each workgroup reads its entry in
 * one load instead of deriving the work split from cached_lens. For engines that run every
 * layer of a decode step over one step's metadata: compute the plan once per step. A plan that
 * does not match the arguments is undefined behaviour (its rows name the sequences, pieces and
 * merges of each workgroup).
 */
hipError_t ie_decode_attention_planned(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,
    const ie_kv_cache* cache, const int32_t* cached_lens, const int32_t* slot_ids,
    const int32_t* num_decoding, const int32_t* plan, int64_t plan_rows, float scale,
    ie_bf16* out, int64_t out_stride_b, int64_t out_stride_h, void* workspace,
    size_t workspace_bytes, hipStream_t stream);
hipError_t ie_decode_attention_rope_planned(
    const ie_bf16* q, int64_t q_stride_b, int64_t q_stride_h, const ie_bf16* k,
    int64_t k_stride_b, int64_t k_stride_h, const ie_bf16* v, int64_t v_stride_b,
    int64_t v_stride_h, const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
    const ie_bf16* cos, int64_t cos_stride_b, const ie_bf16* sin, int64_t sin_stride_b,
    float eps, int32_t batch, int32_t num_q_heads, const ie_kv_cache* cache,
    const int32_t* cached_lens, const int32_t* slot_ids, const int32_t* num_decoding,
    const int32_t* plan, int64_t plan_rows, float scale, ie_bf16* out, int64_t out_stride_b,
    int64_t out_stride_h, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Prefill-side q/k RMSNorm + RoPE over packed tokens.
 * Replaces qwen3-1.7b/kernels.py:665-714 `fused_norm_rope_prefill(q, k, q_norm_weight,
 * k_norm_weight, cos, sin, eps) -> (q_out, k_out)` (kernel kernels.py:547-662).
 *
 * q: bf16 [N, num_q_heads, head_dim], k: bf16 [N, num_kv_heads, head_dim], any token/head
 * strides with unit channel stride (views of the fused qkv output); weights bf16 [head_dim];
 * cos, sin: bf16 [N, 1, head_dim / 2] with unit channel stride. For every token and head row x:
 * x <- x * rstd * w with rstd exactly as in ie_fused_rope_kv_decode (butterfly sum of squares,
 * IEEE 1 / sqrt), then (x1, x2) <- (x1 c - x2 s, x1 s + x2 c) over the two halves; q_out /
 * k_out get the bf16 result (round to nearest even). head_dim must be 128.
 */
hipError_t ie_fused_norm_rope_prefill(const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head,
                                      const ie_bf16* k, int64_t k_stride_tok, int64_t k_stride_head,
                                      const ie_bf16* q_norm_weight, const ie_bf16* k_norm_weight,
                                      const ie_bf16* cos, int64_t cos_stride_tok,
                                      const ie_bf16* sin, int64_t sin_stride_tok,
                                      int64_t num_tokens, int32_t num_q_heads,
                                      int32_t num_kv_heads, int32_t head_dim, float eps,
                                      ie_bf16* q_out, int64_t q_out_stride_tok,
                                      int64_t q_out_stride_head, ie_bf16* k_out,
                                      int64_t k_out_stride_tok, int64_t k_out_stride_head,
                                      hipStream_t stream);

/*
 * int8 cache prefix -> bf16 (k = bf16((q * k_scale) * cal), v = bf16(q * v_scale)).
 * Replaces qwen3-1.7b/kernels.py:935-970 `dequantize_kv_prefix(cache, cu_cached, slot_ids,
 * k_out, v_out)` (kernel kernels.py:868-932). Entry b's prefix, cache row slot_ids[b] columns
 * [0, cu_cached[b+1] - cu_cached[b]), goes to rows [cu_cached[b], cu_cached[b+1]) of
 * k_out/v_out: bf16 [num_kv_heads, >= total, head_dim].
 */
hipError_t ie_dequantize_kv_prefix(const ie_kv_cache* cache, const int32_t* cu_cached,
                                   const int32_t* slot_ids, int32_t num_entries,
                                   ie_bf16* k_out, ie_bf16* v_out, int64_t out_stride_head,
                                   int64_t out_stride_tok, hipStream_t stream);

/*
 * Causal chunked-prefill attention that reads each entry's cached prefix straight from the int8
 * cache and runs QK^T and PV on bf16 MFMA: prefix V is dequantized in LDS with the rounding of
 * ie_dequantize_kv_prefix, prefix K is staged as exact integers with its scale and calibration
 * folded into the scores and into q. Any GQA ratio num_q_heads / num_kv_heads of 1 to 16,
 * head_dim 128; a workgroup serves one pair of a KV head's query heads.
 * Replaces qwen3-1.7b/kernels.py:1129-1175 `prefill_attention(q, k, v, seq_ids, cu_seqlens,
 * tile_start, k_prefix, v_prefix, cu_cached, PREFILL_BLOCK_M)` (kernel kernels.py:987-1126)
 * together with the dequantize_kv_prefix call that fed it (qwen3-1.7b/architecture.py:151-170):
 * the bf16 prefix buffers are replaced by (cache, slot_ids).
 *
 * q: bf16 [N, num_q_heads, head_dim]; k, v: bf16 [N, num_kv_heads, head_dim] (the new chunk,
 * strided views allowed); tile_start: int32 [num_tiles], first packed row of each tile of
 * block_m rows, -1 = no work; every tile lies inside one entry. Row m of entry e attends to the
 * e's prefix (cache row slot_ids[e], columns [0, cu_cached[e+1] - cu_cached[e])) and to its own
 * chunk rows [cu_seqlens[e], m]. Rows of out that no tile covers are left untouched.
 * num_entries = the length of slot_ids (cu_seqlens and cu_cached hold num_entries + 1), any
 * count >= 1. Up to 512 entries a tile's entry is found by binary search over cu_seqlens
 * (the tables staged on chip) and seq_ids is not read; above 512 it is seq_ids[first row of the
 * tile], as in the reference kernel (kernels.py:1029), and seq_ids must hold num_tokens values.
 * Long key ranges are split across workgroups, and the last piece of a split range to finish
 * merges the pieces in the same launch. `workspace` must hold
 * ie_prefill_attention_workspace_size(num_tiles, block_m, num_kv_heads) bytes, a size that
 * depends on the current device's CU count only: one arrival count per resident workgroup
 * (padded to 256 bytes), then the split pieces' partials. The counts must be zero the first
 * time a workspace is used (allocate it zeroed); every launch leaves them zero, so one
 * workspace serves every call in stream order. Calls that overlap on one workspace race.
 */
size_t ie_prefill_attention_workspace_size(int32_t num_tiles, int32_t block_m,
                                           int32_t num_kv_heads);
/* The leading bytes of a prefill workspace that must be zero on entry (the arrival and finish
 * words, two uint32 per resident workgroup, padded to 256 bytes); as for
 * ie_decode_attention_workspace_counts_bytes. No counterpart in the reference. */
size_t ie_prefill_attention_workspace_counts_bytes(void);
hipError_t ie_prefill_attention(const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const ie_bf16* k, int64_t k_stride_tok, int64_t k_stride_head,
                                const ie_bf16* v, int64_t v_stride_tok, int64_t v_stride_head,
                                int64_t num_tokens, int32_t num_q_heads,
                                const int32_t* seq_ids, const int32_t* cu_seqlens,
                                const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
                                const ie_kv_cache* cache, const int32_t* slot_ids,
                                const int32_t* cu_cached, int32_t num_entries, ie_bf16* out,
                                int64_t out_stride_tok,
                                int64_t out_stride_head, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

/*
 * The prefill launch's work list (no counterpart in the reference, whose prefill grid is one
 * program per (tile, query head), kernels.py:1146-1150):
 * ie_prefill_attention_grid(num_tiles, block_m, num_q_heads, num_kv_heads) is the launch's
 * workgroup count, and ie_prefill_attention_plan writes, for each workgroup w, 16 int32 at
 * rows[16 w]:
 *   found, sub-block, unit, piece, pieces of its (sub-block, unit) pair, first tile, end tile,
 *   prefix tiles, chunk tiles, first row, end row, the entry's first row, prefix length, cache
 *   slot, straddling form (1) or separate prefix/chunk pieces (0), the pair's first item
 * where sub-blocks are 128-row slices of the tiles, a unit is a KV head and one pair of its
 * query heads (unit = KV head * cdiv(ratio, 2) + pair: the KV head itself at GQA ratio 2), tile
 * t < prefix tiles is the prefix's 64-key tile t and later tiles are the chunk's 64-key tiles,
 * and a workgroup without work has an all-zero row. Same index arguments as
 * ie_prefill_attention; rows: int32 [grid, 16] device memory. The list depends on the index
 * arrays' values, the head counts and the device's CU count only, so one list serves every
 * layer of a step.
 */
int32_t ie_prefill_attention_grid(int32_t num_tiles, int32_t block_m, int32_t num_q_heads,
                                  int32_t num_kv_heads);
hipError_t ie_prefill_attention_plan(const int32_t* seq_ids, const int32_t* cu_seqlens,
                                     const int32_t* tile_start, int32_t num_tiles,
                                     int32_t block_m, int64_t num_tokens, int32_t num_q_heads,
                                     int32_t num_kv_heads, const int32_t* slot_ids,
                                     const int32_t* cu_cached, int32_t num_entries, int32_t* rows,
                                     hipStream_t stream);
/*
 * ie_prefill_attention with its work list precomputed (no counterpart in the reference): the
 * same arguments and results, plus `plan`, the rows ie_prefill_attention_plan wrote for the
 * same index arrays (same values), head counts, block_m and device, and plan_rows, their count
 * (at least the grid). Each workgroup then reads its row in one load instead of deriving the
 * list from the tile metadata, which every workgroup of ie_prefill_attention does. The index
 * arrays are not read. For engines that run several layers over one step's metadata: compute
 * the plan once per step. A plan that does not match the arguments is undefined behaviour (its
 * rows name the cache slots, rows and tiles each workgroup reads and writes).
 */
hipError_t ie_prefill_attention_planned(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached,
    int32_t num_entries, const int32_t* plan, int64_t plan_rows, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    hipStream_t stream);

/*
 * Token sampling: Gumbel-max over the vocabulary, greedy argmax at tau = 0.
 * Replaces qwen3-1.7b/kernels.py:1343-1370 `sample(logits, tau, seed) -> [B, 1] int64`
 * (kernels sampling_kernel :1286-1318 and combine_partial_samples_kernel :1321-1340).
 *
 * logits: [batch, vocab] of logits_dtype (IE_DTYPE_BF16 or IE_DTYPE_F32), unit stride along the
 * vocabulary, row stride logits_stride_row elements. out[b * out_stride_row] = the first v that
 * maximizes logits[b, v] + tau * -log(-log(clamp(u, 1e-10, 1 - 1e-7))), where u is Triton's
 * tl.rand(seed, b * vocab + v): Philox4x32-10 on counter (b * vocab + v as int32, 0, 0, 0) and
 * key (low, high 32 bits of *seed), first output word x as int32,
 * u = float(x < 0 ? -x - 1 : x) * 4.6566127342e-10. At tau = 0 no uniform is drawn. *seed (a
 * device int64) is incremented once per call, after every row has read it, also when batch is
 * 0. `workspace` must hold ie_sample_workspace_size(batch, vocab) bytes.
 */
size_t ie_sample_workspace_size(int32_t batch, int64_t vocab);
hipError_t ie_sample(const void* logits, int32_t logits_dtype, int64_t logits_stride_row,
                     int32_t batch, int64_t vocab, float tau, int64_t* seed, int64_t* out,
                     int64_t out_stride_row, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/*
 * Residual add + RMSNorm of token rows.
 * Replaces qwen3-1.7b/kernels.py:1260-1283 `add_rms_norm(residual, delta, rms_norm, eps) ->
 * (new_residual, new_normed_residual)` (kernel kernels.py:1216-1257).
 *
 * residual, delta, new_residual, normed: bf16 [num_tokens, dim] rows (any row strides, 16-byte
 * aligned rows); weight: bf16 [dim]; dim a multiple of 8, at most 8192. new_residual =
 * bf16(residual + delta); normed = bf16((r * rstd) * w) with r = new_residual and
 * rstd = 1 / sqrt(sum(r^2) / dim + eps) (IEEE). Sum order: thread t of 256 adds the squares of
 * elements 8t + 2048j + i in order, the wave's 64 sums combine by the xor butterfly (lane
 * distance 32 ... 1), the four wave sums are added in order.
 */
hipError_t ie_add_rms_norm(const ie_bf16* residual, int64_t residual_stride, const ie_bf16* delta,
                           int64_t delta_stride, const ie_bf16* weight, int64_t num_tokens,
                           int32_t dim, float eps, ie_bf16* new_residual,
                           int64_t new_residual_stride, ie_bf16* normed, int64_t normed_stride,
                           hipStream_t stream);

/*
 * RoPE tables of a step's positions, for the q/k RoPE of the other entry points (no separate
 * function in the reference, which computes them with PyTorch at architecture.py:382-390):
 * cos_out[t, j] = bf16(cos(float(positions[t]) * inv_freq[j])), sin_out likewise, for t < n,
 * j < half_dim (one fp32 product, the device library's cosf/sinf, round to nearest even);
 * outputs [n, half_dim] contiguous (the [n, 1, head_dim / 2] tables the kernels take).
 */
hipError_t ie_rope_tables(const int32_t* positions, int64_t n, const float* inv_freq,
                          int32_t half_dim, ie_bf16* cos_out, ie_bf16* sin_out,
                          hipStream_t stream);

/*
 * SiLU-gated product. Replaces qwen3-1.7b/kernels.py:1204-1213 `silu_mul(gate_up) -> out`
 * (kernel kernels.py:1178-1201): gate_up bf16 [num_tokens, 2 * dim] (gate then up), out bf16
 * [num_tokens, dim] = bf16((g * sigmoid(g)) * u), sigmoid(g) = 1 / (1 + exp(-g)) in fp32.
 * dim a multiple of 8, rows 16-byte aligned.
 */
hipError_t ie_silu_mul(const ie_bf16* gate_up, int64_t gate_up_stride, int64_t num_tokens,
                       int32_t dim, ie_bf16* out, int64_t out_stride, hipStream_t stream);

/*
 * y = x . weight^T for few rows (decode). Replaces qwen3-1.7b/kernels.py:1406-1443
 * `skinny_matmul(x, weight) -> y` (kernel kernels.py:1373-1403), which `linear`
 * (kernels.py:1451-1458) picks per (N, K, M) over the library GEMM after `tune_linear` timed both.
 * x: bf16 [m, k] (m <= 64), weight: bf16 [n, k] (nn.Linear layout), y: bf16 [m, n]; fp32
 * accumulation, y rounded to nearest even. n_tiles (1, 2 or 4): weight rows per workgroup / 16,
 * or 0 for 8 rows per workgroup, the shape-dependent launch choice (more rows per workgroup
 * re-read x less often, fewer workgroups fill fewer CUs; it is lowered where m leaves too little
 * LDS for it, which can change the rounding of the k summation, not the result's tolerance).
 * n a multiple of 16 max(1, n_tiles), k of 256; rows 16-byte aligned (y 8-byte).
 */
hipError_t ie_skinny_gemm(const ie_bf16* x, int64_t x_stride, int32_t m, const ie_bf16* weight,
                          int64_t weight_stride, int32_t n, int32_t k, int32_t n_tiles, ie_bf16* y,
                          int64_t y_stride, hipStream_t stream);

/*
 * y = silu_mul(x . weight^T) in one launch: the MLP's gate/up projection followed by the
 * SiLU-gated product, i.e. qwen3-1.7b/kernels.py:1451-1458 `linear(x, w_gate_up)` then
 * kernels.py:1178-1213 `silu_mul` (called in sequence at architecture.py:282-300). weight: bf16
 * [n, k], the n / 2 gate rows then the n / 2 up rows; y: bf16 [m, n / 2] =
 * bf16((g * (1 / (1 + e^-g))) * u) with g, u the bf16-rounded products, as the two-step path
 * computes them (the products' fp32 summation order may differ from ie_skinny_gemm's, within
 * its tolerance). n_tiles (1 or 2): gate (and up) rows per workgroup / 16, lowered to 1 where m
 * leaves too little LDS. n / 2 a multiple of 16 n_tiles, k of 256; m <= 64.
 */
hipError_t ie_skinny_gemm_silu_mul(const ie_bf16* x, int64_t x_stride, int32_t m,
                                   const ie_bf16* weight, int64_t weight_stride, int32_t n,
                                   int32_t k, int32_t n_tiles, ie_bf16* y, int64_t y_stride,
                                   hipStream_t stream);

/*
 * The skinny GEMM with a decoder layer's residual add and RMSNorm fused in (no counterpart in
 * the reference, whose block calls add_rms_norm between its projections, kernels.py:1260-1283
 * at architecture.py:280-300): for engines that fold each RMSNorm's weight into the weight
 * columns of the projections it feeds, which removes both add_rms_norm launches of a layer.
 * flags:
 *   0                 y = x . weight^T (ie_skinny_gemm);
 *   IE_SKINNY_SILU_MUL   the gate/up form of ie_skinny_gemm_silu_mul;
 *   IE_SKINNY_NORM    x is the residual stream h (new_residual of add_rms_norm) and weight holds
 *                     bf16(W[n, k] * g[k]) for the norm weight g: every fp32 sum of row m is
 *                     multiplied by rstd_m = 1 / sqrt(sum_k h[m, k]^2 / k + eps) (IEEE) before
 *                     it is rounded, i.e. the GEMM of RMSNorm(h) * g up to where the rounding
 *                     to bf16 falls (the weight is rounded after the product with g instead of
 *                     the normalized row); combines with IE_SKINNY_SILU_MUL;
 *   IE_SKINNY_RESIDUAL   y holds the residual stream on entry and becomes
 *                     bf16(y + bf16(x . weight^T)) in place: add_rms_norm's new_residual for the
 *                     projection's output as delta, bit for bit (x must not overlap y).
 *   | IE_SKINNY_SWIZZLED (with any of the above) weight is the output of
 *                     ie_skinny_weight_swizzle for this n_tiles (1, 2 or 4; weight_stride = k;
 *                     an n_tiles too wide for m is an error, not lowered): the same results, bit
 *                     for bit, as the row-major weight with the same n_tiles; with
 *                     IE_SKINNY_SILU_MUL, the output of ie_skinny_weight_swizzle_gate_up for this
 *                     n_tiles (1 ... 4, 8 n_tiles output columns per workgroup): for even n_tiles
 *                     the row-major gate/up form's results at n_tiles / 2, bit for bit;
 *   | IE_SKINNY_Y_FRAGMENTS (the swizzled gate/up form; y_stride = n / 2, n / 2 a multiple of
 *                     32) y is written in MFMA fragment order: y holds cdiv(m, 16) * 16 x n / 2
 *                     bf16 as 1 KB blocks, block S * cdiv(m, 16) + t for column step S (columns
 *                     32 S .. 32 S + 31) and row tile t, holding at byte 16 (16 g + r) row
 *                     16 t + r, columns 32 S + 8 g .. 32 S + 8 g + 7 (rows past m not written);
 *   | IE_SKINNY_X_FRAGMENTS (the plain or residual form; x_stride = k) x is in that order (the
 *                     y of an IE_SKINNY_Y_FRAGMENTS call with the same m), read as contiguous
 *                     1 KB blocks without the LDS round trip: the same results, bit for bit.
 * Sizes, strides and n_tiles as for the plain or the gate/up form. The sum of squares is taken
 * from the bf16 rows of x over all k columns (eight partial sums combined in a fixed order).
 */
#define IE_SKINNY_NORM 1
#define IE_SKINNY_SILU_MUL 2
#define IE_SKINNY_RESIDUAL 4
#define IE_SKINNY_SWIZZLED 8
#define IE_SKINNY_X_FRAGMENTS 16
#define IE_SKINNY_Y_FRAGMENTS 32
hipError_t ie_skinny_gemm_fused(const ie_bf16* x, int64_t x_stride, int32_t m,
                                const ie_bf16* weight, int64_t weight_stride, int32_t n, int32_t k,
                                int32_t n_tiles, int32_t flags, float eps, ie_bf16* y,
                                int64_t y_stride, hipStream_t stream);

/*
 * A weight's elements in the order the skinny GEMM's waves consume them for a tile width
 * n_tiles (1, 2 or 4) (no counterpart in the reference; for weights used many times, e.g. every
 * decode step's projections, reordered once at load): out holds n x k bf16, as 1 KB blocks,
 * block ((R / G) * k / 32 + S) * G + R % G (G = n_tiles) for row group R (rows 16 R .. 16 R +
 * 15) and column step S (columns 32 S .. 32 S + 31), each holding, at byte 16 (16 g + r), row
 * 16 R + r, columns 32 S + 8 g .. 32 S + 8 g + 7 (each workgroup's G groups interleaved step by
 * step). With it a wave reads an MFMA operand fragment as one contiguous 1 KB load instead of
 * staging row-major rows through LDS; the GEMM must take the same n_tiles. weight: bf16 [n, k]
 * rows (16-byte aligned, stride weight_stride); n a multiple of 16 n_tiles, k of 32.
 */
hipError_t ie_skinny_weight_swizzle(const ie_bf16* weight, int64_t weight_stride, int32_t n,
                                    int32_t k, int32_t n_tiles, ie_bf16* out,
                                    hipStream_t stream);

/*
 * The LM head and greedy sampling in one launch (no counterpart in the reference, which runs
 * kernels.py:1451-1458 `linear` then kernels.py:1343-1370 `sample` at tau = 0): logits =
 * ie_skinny_gemm_fused(x, weight, flags) (flags 0 or IE_SKINNY_NORM; weight swizzled for
 * n_tiles 1, 2 or 4, k = 2048, on one looping workgroup per CU: the same logits bits as that
 * call), tokens[r * tokens_stride] = the first column of the largest logit of row r (sample's
 * greedy choice on these logits, NaN never chosen, 0x7fffffff for an all-NaN row), and *seed
 * advanced by one as sample advances it. workspace: ie_skinny_lm_head_greedy_workspace_size()
 * bytes, 16-byte aligned, zero before the first call (every call leaves it zero); calls that
 * overlap on one workspace race. m <= 64.
 */
size_t ie_skinny_lm_head_greedy_workspace_size(void);
hipError_t ie_skinny_lm_head_greedy(const ie_bf16* x, int64_t x_stride, int32_t m,
                                    const ie_bf16* weight, int32_t n, int32_t k, int32_t n_tiles,
                                    int32_t flags, float eps, ie_bf16* logits,
                                    int64_t logits_stride, int64_t* tokens, int64_t tokens_stride,
                                    int64_t* seed, void* workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/*
 * The gate/up weight of ie_skinny_gemm_silu_mul (n / 2 gate rows, then the n / 2 up rows) in the
 * order of ie_skinny_weight_swizzle after pairing its rows (no counterpart in the reference):
 * 16-row group R holds gate rows 8 R .. 8 R + 7, then up rows n / 2 + 8 R .. n / 2 + 8 R + 7, so
 * one MFMA tile yields 8 gate sums and their 8 up sums. For ie_skinny_gemm_fused with
 * IE_SKINNY_SILU_MUL | IE_SKINNY_SWIZZLED and the same n_tiles (1, 2, 3 or 4; n a multiple of
 * 16 n_tiles, k of 32).
 */
hipError_t ie_skinny_weight_swizzle_gate_up(const ie_bf16* weight, int64_t weight_stride,
                                            int32_t n, int32_t k, int32_t n_tiles, ie_bf16* out,
                                            hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* IE_ATTN_H */
