// torch.ops.ie.* registration: validates tensors, turns them into the plain pointers, strides and
// sizes of the C ABI (include/ie_attn.h), and enqueues on the current HIP stream. No kernel
// code lives here and nothing is computed on the host; workspaces come from the PyTorch
// caching allocator (the graph pool while a hipGraph is being captured).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <map>
#include <tuple>
#include <mutex>
#include <vector>

#include "../../include/ie_attn.h"

namespace {

void ok(hipError_t e, const char* what) {
    TORCH_CHECK(e == hipSuccess, "ie.", what, ": ", hipGetErrorString(e), " (",
                ie_attn_last_error(), ")");
}

hipStream_t stream_of(const at::Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_dev(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), "ie: ", name, " must be a GPU tensor");
}

void check_i32(const at::Tensor& t, const char* name) {
    check_dev(t, name);
    TORCH_CHECK(t.scalar_type() == at::kInt, "ie: ", name, " must be int32");
    TORCH_CHECK(t.dim() == 1 && t.stride(0) == 1, "ie: ", name, " must be a contiguous vector");
}

void check_bf16_rows(const at::Tensor& t, const char* name, int64_t dim) {
    check_dev(t, name);
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, "ie: ", name, " must be bfloat16");
    TORCH_CHECK(t.dim() == dim, "ie: ", name, " must have ", dim, " dims");
    TORCH_CHECK(t.stride(-1) == 1, "ie: ", name, " needs a contiguous last dim");
}

const ie_bf16* bf(const at::Tensor& t) {
    return reinterpret_cast<const ie_bf16*>(t.data_ptr());
}
ie_bf16* bfm(const at::Tensor& t) { return reinterpret_cast<ie_bf16*>(t.data_ptr()); }
const int32_t* i32(const at::Tensor& t) { return t.data_ptr<int32_t>(); }
int32_t* i32m(const at::Tensor& t) { return t.data_ptr<int32_t>(); }

// LayerKVCache (qwen3-1.7b/kernels.py:11-17) -> descriptor; same stride asserts as
// kernels.py:284-287.
ie_kv_cache cache_desc(const at::Tensor& k, const at::Tensor& v, const at::Tensor& ks,
                       const at::Tensor& vs, const at::Tensor& cal) {
    check_dev(k, "k_cache");
    TORCH_CHECK(k.scalar_type() == at::kChar && v.scalar_type() == at::kChar,
                "ie: k/v cache must be int8");
    TORCH_CHECK(ks.scalar_type() == at::kFloat && vs.scalar_type() == at::kFloat &&
                    cal.scalar_type() == at::kFloat,
                "ie: scales and calibration must be float32");
    TORCH_CHECK(k.dim() == 4 && v.sizes() == k.sizes(), "ie: k/v cache must be [pool,Hkv,L,D]");
    TORCH_CHECK(k.strides() == v.strides(), "kernel uses one set of strides for k and v");
    TORCH_CHECK(ks.dim() == 3 && vs.sizes() == ks.sizes() && ks.strides() == vs.strides(),
                "ie: k_scale/v_scale must be [pool,Hkv,L] with equal strides");
    TORCH_CHECK(ks.size(0) == k.size(0) && ks.size(1) == k.size(1) && ks.size(2) == k.size(2) &&
                    ks.stride(2) == 1,
                "ie: scale shape/stride mismatch");
    TORCH_CHECK(cal.dim() == 4 && cal.size(0) == k.size(0) && cal.size(1) == k.size(1) &&
                    cal.size(3) == k.size(3) && cal.stride(3) == 1,
                "ie: k_calibration must be [pool,Hkv,1,D]");
    ie_kv_cache c;
    c.k = k.data_ptr<int8_t>();
    c.v = v.data_ptr<int8_t>();
    c.k_scale = ks.data_ptr<float>();
    c.v_scale = vs.data_ptr<float>();
    c.k_calibration = cal.data_ptr<float>();
    c.pool = k.size(0);
    c.num_kv_heads = k.size(1);
    c.max_len = k.size(2);
    c.head_dim = k.size(3);
    c.stride_slot = k.stride(0);
    c.stride_head = k.stride(1);
    c.stride_tok = k.stride(2);
    c.scale_stride_slot = ks.stride(0);
    c.scale_stride_head = ks.stride(1);
    c.cal_stride_slot = cal.stride(0);
    c.cal_stride_head = cal.stride(1);
    TORCH_CHECK(k.stride(3) == 1, "ie: cache head_dim must be contiguous");
    return c;
}

void quantize_kv_prefill(const at::Tensor& k, const at::Tensor& v, const at::Tensor& cu_seqlens,
                         const at::Tensor& slot_ids, const at::Tensor& cached_lens,
                         const at::Tensor& num_decoding, const at::Tensor& k_cache,
                         const at::Tensor& v_cache, const at::Tensor& k_scale,
                         const at::Tensor& v_scale, const at::Tensor& k_calibration) {
    check_bf16_rows(k, "k", 3);
    check_bf16_rows(v, "v", 3);
    for (auto* t : {&cu_seqlens, &slot_ids, &cached_lens, &num_decoding}) check_i32(*t, "index");
    const c10::DeviceGuard guard(k.device());
    ie_kv_cache c = cache_desc(k_cache, v_cache, k_scale, v_scale, k_calibration);
    TORCH_CHECK(k.size(1) == c.num_kv_heads && k.size(2) == c.head_dim && v.sizes() == k.sizes(),
                "ie: k/v shape mismatch");
    const int32_t entries = (int32_t)cu_seqlens.size(0) - 1;
    TORCH_CHECK(slot_ids.size(0) >= entries && cached_lens.size(0) >= entries,
                "ie: slot_ids/cached_lens shorter than the entry count");
    ok(ie_quantize_kv_prefill(bf(k), k.stride(0), k.stride(1), bf(v), v.stride(0), v.stride(1),
                              k.size(0), i32(cu_seqlens), i32(slot_ids), i32(cached_lens),
                              i32(num_decoding), entries, &c, stream_of(k)),
       "quantize_kv_prefill");
}

at::Tensor fused_rope_kv_decode(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                const at::Tensor& q_norm_weight,
                                const at::Tensor& k_norm_weight, const at::Tensor& cos,
                                const at::Tensor& sin, const at::Tensor& slot_ids,
                                const at::Tensor& k_cache, const at::Tensor& v_cache,
                                const at::Tensor& k_scale, const at::Tensor& v_scale,
                                const at::Tensor& k_calibration, const at::Tensor& cached_lens,
                                const at::Tensor& num_decoding, double eps) {
    check_bf16_rows(q, "q", 3);
    check_bf16_rows(k, "k", 3);
    check_bf16_rows(v, "v", 3);
    check_bf16_rows(q_norm_weight, "q_norm_weight", 1);
    check_bf16_rows(k_norm_weight, "k_norm_weight", 1);
    check_bf16_rows(cos, "cos", 3);
    check_bf16_rows(sin, "sin", 3);
    for (auto* t : {&slot_ids, &cached_lens, &num_decoding}) check_i32(*t, "index");
    const c10::DeviceGuard guard(q.device());
    ie_kv_cache c = cache_desc(k_cache, v_cache, k_scale, v_scale, k_calibration);
    const int64_t B = q.size(0), hq = q.size(1);
    TORCH_CHECK(q.size(2) == 128 && k.size(2) == 128 && v.size(2) == 128, "ie: head_dim 128");
    TORCH_CHECK(k.size(0) >= B && v.size(0) >= B && k.size(1) == c.num_kv_heads &&
                    v.size(1) == c.num_kv_heads,
                "ie: k/v shape mismatch");
    TORCH_CHECK(cos.size(0) >= B && sin.size(0) >= B && cos.size(2) == 64 && sin.size(2) == 64,
                "ie: cos/sin must be [B,1,64]");
    TORCH_CHECK(slot_ids.size(0) >= B && cached_lens.size(0) >= B, "ie: index tensors too short");
    at::Tensor out = at::empty({B, hq, 128}, q.options());
    ok(ie_fused_rope_kv_decode(bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1),
                               bf(v), v.stride(0), v.stride(1), bf(q_norm_weight),
                               bf(k_norm_weight), bf(cos), cos.stride(0), bf(sin), sin.stride(0),
                               i32(slot_ids), i32(cached_lens), i32(num_decoding), (int32_t)B,
                               (int32_t)hq, (float)eps, &c, bfm(out), out.stride(0),
                               out.stride(1), stream_of(q)),
       "fused_rope_kv_decode");
    return out;
}

std::tuple<at::Tensor, at::Tensor> fused_norm_rope_prefill(const at::Tensor& q,
                                                           const at::Tensor& k,
                                                           const at::Tensor& q_norm_weight,
                                                           const at::Tensor& k_norm_weight,
                                                           const at::Tensor& cos,
                                                           const at::Tensor& sin, double eps) {
    check_bf16_rows(q, "q", 3);
    check_bf16_rows(k, "k", 3);
    check_bf16_rows(q_norm_weight, "q_norm_weight", 1);
    check_bf16_rows(k_norm_weight, "k_norm_weight", 1);
    check_bf16_rows(cos, "cos", 3);
    check_bf16_rows(sin, "sin", 3);
    const c10::DeviceGuard guard(q.device());
    const int64_t N = q.size(0), hq = q.size(1), hkv = k.size(1), D = q.size(2);
    TORCH_CHECK(D == 128 && k.size(2) == D, "ie: head_dim 128");
    TORCH_CHECK(k.size(0) == N && cos.size(0) >= N && sin.size(0) >= N && cos.size(2) == D / 2 &&
                    sin.size(2) == D / 2,
                "ie: k [N, Hkv, D], cos/sin [N, 1, D/2]");
    TORCH_CHECK(q_norm_weight.size(0) == D && k_norm_weight.size(0) == D, "ie: norm weights [D]");
    at::Tensor q_out = at::empty({N, hq, D}, q.options());
    at::Tensor k_out = at::empty({N, hkv, D}, k.options());
    ok(ie_fused_norm_rope_prefill(bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1),
                                  bf(q_norm_weight), bf(k_norm_weight), bf(cos), cos.stride(0),
                                  bf(sin), sin.stride(0), N, (int32_t)hq, (int32_t)hkv,
                                  (int32_t)D, (float)eps, bfm(q_out), q_out.stride(0),
                                  q_out.stride(1), bfm(k_out), k_out.stride(0), k_out.stride(1),
                                  stream_of(q)),
       "fused_norm_rope_prefill");
    return {q_out, k_out};
}

at::Tensor sample(const at::Tensor& logits, double tau, const at::Tensor& seed) {
    TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.stride(1) == 1,
                "ie: logits must be a [B, V] device tensor with unit vocab stride");
    TORCH_CHECK(logits.scalar_type() == at::kBFloat16 || logits.scalar_type() == at::kFloat,
                "ie: logits must be bf16 or fp32");
    TORCH_CHECK(seed.is_cuda() && seed.scalar_type() == at::kLong && seed.numel() >= 1 &&
                    seed.is_contiguous(),
                "ie: seed must be an int64 device tensor");
    const c10::DeviceGuard guard(logits.device());
    const int64_t B = logits.size(0), V = logits.size(1);
    at::Tensor out = at::empty({B, 1}, logits.options().dtype(at::kLong));
    const size_t ws_bytes = ie_sample_workspace_size((int32_t)B, V);
    at::Tensor ws = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)},
                              logits.options().dtype(at::kByte));
    ok(ie_sample(logits.data_ptr(),
                 logits.scalar_type() == at::kBFloat16 ? IE_DTYPE_BF16 : IE_DTYPE_F32,
                 logits.stride(0), (int32_t)B, V, (float)tau, seed.data_ptr<int64_t>(),
                 out.data_ptr<int64_t>(), out.stride(0), ws.data_ptr(), ws_bytes,
                 stream_of(logits)),
       "sample");
    return out;
}

std::tuple<at::Tensor, at::Tensor> add_rms_norm(const at::Tensor& residual,
                                                const at::Tensor& delta,
                                                const at::Tensor& weight, double eps) {
    check_bf16_rows(residual, "residual", 2);
    check_bf16_rows(delta, "delta", 2);
    check_bf16_rows(weight, "weight", 1);
    const c10::DeviceGuard guard(residual.device());
    const int64_t N = residual.size(0), D = residual.size(1);
    TORCH_CHECK(delta.size(0) == N && delta.size(1) == D && weight.size(0) == D,
                "ie: residual/delta [N, D], weight [D]");
    at::Tensor nres = at::empty({N, D}, residual.options());
    at::Tensor normed = at::empty({N, D}, residual.options());
    ok(ie_add_rms_norm(bf(residual), residual.stride(0), bf(delta), delta.stride(0), bf(weight), N,
                       (int32_t)D, (float)eps, bfm(nres), nres.stride(0), bfm(normed),
                       normed.stride(0), stream_of(residual)),
       "add_rms_norm");
    return {nres, normed};
}

// RoPE tables of int32 positions [N] and fp32 inv_freq [D / 2]: bf16 cos, sin [N, 1, D / 2].
std::tuple<at::Tensor, at::Tensor> rope_tables(const at::Tensor& positions,
                                               const at::Tensor& inv_freq) {
    check_i32(positions, "positions");
    check_dev(inv_freq, "inv_freq");
    TORCH_CHECK(inv_freq.scalar_type() == at::kFloat && inv_freq.dim() == 1 &&
                    inv_freq.is_contiguous() && inv_freq.device() == positions.device(),
                "ie: inv_freq must be a contiguous fp32 vector on the positions' device");
    const c10::DeviceGuard guard(positions.device());
    const int64_t N = positions.size(0), H = inv_freq.size(0);
    auto opt = positions.options().dtype(at::kBFloat16);
    at::Tensor c = at::empty({N, 1, H}, opt), s = at::empty({N, 1, H}, opt);
    ok(ie_rope_tables(i32(positions), N, inv_freq.data_ptr<float>(), (int32_t)H, bfm(c), bfm(s),
                      stream_of(positions)),
       "rope_tables");
    return {c, s};
}

at::Tensor silu_mul(const at::Tensor& gate_up) {
    check_bf16_rows(gate_up, "gate_up", 2);
    const c10::DeviceGuard guard(gate_up.device());
    const int64_t N = gate_up.size(0), D = gate_up.size(1) / 2;
    TORCH_CHECK(gate_up.size(1) % 2 == 0, "ie: gate_up must be [N, 2D]");
    at::Tensor out = at::empty({N, D}, gate_up.options());
    ok(ie_silu_mul(bf(gate_up), gate_up.stride(0), N, (int32_t)D, bfm(out), out.stride(0),
                   stream_of(gate_up)),
       "silu_mul");
    return out;
}

// A weight from skinny_weight_swizzle: a contiguous [N, K] bf16 tensor in fragment order.
void check_swizzled(const at::Tensor& weight, bool swizzled) {
    TORCH_CHECK(!swizzled || weight.is_contiguous(),
                "ie: a swizzled weight is the contiguous output of skinny_weight_swizzle");
}

at::Tensor skinny_matmul(const at::Tensor& x, const at::Tensor& weight, int64_t n_tiles,
                         bool swizzled) {
    check_bf16_rows(x, "x", 2);
    check_bf16_rows(weight, "weight", 2);
    check_swizzled(weight, swizzled);
    const c10::DeviceGuard guard(x.device());
    const int64_t M = x.size(0), K = x.size(1), N = weight.size(0);
    TORCH_CHECK(weight.size(1) == K, "ie: weight must be [N, K]");
    at::Tensor y = at::empty({M, N}, x.options());
    ok(ie_skinny_gemm_fused(bf(x), x.stride(0), (int32_t)M, bf(weight), weight.stride(0),
                            (int32_t)N, (int32_t)K, (int32_t)n_tiles,
                            swizzled ? IE_SKINNY_SWIZZLED : 0, 0.f, bfm(y), y.stride(0),
                            stream_of(x)),
       "skinny_matmul");
    return y;
}

at::Tensor skinny_matmul_silu_mul(const at::Tensor& x, const at::Tensor& weight, int64_t n_tiles,
                                  bool swizzled) {
    check_bf16_rows(x, "x", 2);
    check_bf16_rows(weight, "weight", 2);
    check_swizzled(weight, swizzled);
    const c10::DeviceGuard guard(x.device());
    const int64_t M = x.size(0), K = x.size(1), N = weight.size(0);
    TORCH_CHECK(weight.size(1) == K, "ie: weight must be [N, K]");
    TORCH_CHECK(N % 2 == 0, "ie: weight must hold the gate rows then the up rows");
    at::Tensor y = at::empty({M, N / 2}, x.options());
    ok(ie_skinny_gemm_fused(bf(x), x.stride(0), (int32_t)M, bf(weight), weight.stride(0),
                            (int32_t)N, (int32_t)K, (int32_t)n_tiles,
                            IE_SKINNY_SILU_MUL | (swizzled ? IE_SKINNY_SWIZZLED : 0), 0.f,
                            bfm(y), y.stride(0), stream_of(x)),
       "skinny_matmul_silu_mul");
    return y;
}

// The weight in the skinny GEMM's fragment order for n_tiles (ie_skinny_weight_swizzle; the
// gate/up weight of the SiLU-gated form in paired order with gate_up,
// ie_skinny_weight_swizzle_gate_up), for swizzled=True calls with the same n_tiles.
at::Tensor skinny_weight_swizzle(const at::Tensor& weight, int64_t n_tiles, bool gate_up) {
    check_bf16_rows(weight, "weight", 2);
    const c10::DeviceGuard guard(weight.device());
    at::Tensor out = at::empty(weight.sizes(), weight.options());
    auto fn = gate_up ? ie_skinny_weight_swizzle_gate_up : ie_skinny_weight_swizzle;
    ok(fn(bf(weight), weight.stride(0), (int32_t)weight.size(0), (int32_t)weight.size(1),
          (int32_t)n_tiles, bfm(out), stream_of(weight)),
       "skinny_weight_swizzle");
    return out;
}

// The GEMM of RMSNorm(h) with the norm weight folded into `weight` (ie_skinny_gemm_fused with
// IE_SKINNY_NORM, and IE_SKINNY_SILU_MUL for the gate/up form; fragments: the swizzled gate/up
// form's output in MFMA fragment order, IE_SKINNY_Y_FRAGMENTS, [cdiv(M, 16) 16, N / 2]).
at::Tensor skinny_matmul_norm(const at::Tensor& h, const at::Tensor& weight, int64_t n_tiles,
                              bool silu_mul, double eps, bool swizzled, bool fragments) {
    check_bf16_rows(h, "h", 2);
    check_bf16_rows(weight, "weight", 2);
    check_swizzled(weight, swizzled);
    const c10::DeviceGuard guard(h.device());
    const int64_t M = h.size(0), K = h.size(1), N = weight.size(0);
    TORCH_CHECK(weight.size(1) == K, "ie: weight must be [N, K]");
    TORCH_CHECK(!silu_mul || N % 2 == 0, "ie: weight must hold the gate rows then the up rows");
    TORCH_CHECK(!fragments || (silu_mul && swizzled),
                "ie: fragment-order output: the swizzled gate/up form");
    at::Tensor y = at::empty({fragments ? (M + 15) / 16 * 16 : M, silu_mul ? N / 2 : N},
                             h.options());
    ok(ie_skinny_gemm_fused(bf(h), h.stride(0), (int32_t)M, bf(weight), weight.stride(0),
                            (int32_t)N, (int32_t)K, (int32_t)n_tiles,
                            IE_SKINNY_NORM | (silu_mul ? IE_SKINNY_SILU_MUL : 0) |
                                (swizzled ? IE_SKINNY_SWIZZLED : 0) |
                                (fragments ? IE_SKINNY_Y_FRAGMENTS : 0),
                            (float)eps,
                            bfm(y), y.stride(0), stream_of(h)),
       "skinny_matmul_norm");
    return y;
}

// residual <- bf16(residual + bf16(x . weight^T)) in place (IE_SKINNY_RESIDUAL; x_fragments: x
// is a fragment-order output of skinny_matmul_norm with the same M, IE_SKINNY_X_FRAGMENTS).
at::Tensor skinny_matmul_residual_(const at::Tensor& x, const at::Tensor& weight, int64_t n_tiles,
                                   at::Tensor residual, bool swizzled, bool x_fragments) {
    check_bf16_rows(x, "x", 2);
    check_bf16_rows(weight, "weight", 2);
    check_swizzled(weight, swizzled);
    check_bf16_rows(residual, "residual", 2);
    const c10::DeviceGuard guard(x.device());
    const int64_t M = residual.size(0), K = x.size(1), N = weight.size(0);
    TORCH_CHECK(x_fragments ? x.size(0) == (M + 15) / 16 * 16 && x.is_contiguous()
                            : x.size(0) == M,
                "ie: x must be [M, K] ([cdiv(M, 16) 16, K] contiguous in fragment order)");
    TORCH_CHECK(weight.size(1) == K, "ie: weight must be [N, K]");
    TORCH_CHECK(residual.size(0) == M && residual.size(1) == N, "ie: residual must be [M, N]");
    TORCH_CHECK(residual.device() == x.device() && weight.device() == x.device(),
                "ie: x, weight and residual must be on one device");
    ok(ie_skinny_gemm_fused(bf(x), x.stride(0), (int32_t)M, bf(weight), weight.stride(0),
                            (int32_t)N, (int32_t)K, (int32_t)n_tiles,
                            IE_SKINNY_RESIDUAL | (swizzled ? IE_SKINNY_SWIZZLED : 0) |
                                (x_fragments ? IE_SKINNY_X_FRAGMENTS : 0),
                            0.f,
                            bfm(residual), residual.stride(0), stream_of(x)),
       "skinny_matmul_residual_");
    return residual;
}

struct DecodeCall {
    ie_kv_cache c;
    int32_t B, hq;
    size_t ws_bytes;
};

// A decode work list from decode_plan: int32 [rows, 4], contiguous, on q's device.
void check_decode_plan(const at::Tensor& plan, const at::Tensor& q) {
    check_dev(plan, "plan");
    TORCH_CHECK(plan.scalar_type() == at::kInt && plan.dim() == 2 && plan.size(1) == 4 &&
                    plan.is_contiguous(),
                "ie: plan must be a contiguous int32 [rows, 4] tensor (decode_plan)");
    TORCH_CHECK(plan.device() == q.device(), "ie: plan must be on q's device");
}

// The kept decode workspace a call uses: calls of up to 1024 sequences and 128 query heads
// share one (their count regions coincide), every larger shape has one of its own.
int32_t decode_ws_kind(const DecodeCall& d) {
    if (d.B <= 1024 && d.hq <= 128) return 0;
    return (int32_t)std::min<int64_t>((int64_t)d.B * 1024 + std::min(d.hq, 1023), INT32_MAX);
}

DecodeCall decode_prep(const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                       const at::Tensor& k_scale, const at::Tensor& v_scale,
                       const at::Tensor& k_calibration, const at::Tensor& cached_lens,
                       const at::Tensor& slot_ids, const at::Tensor& num_decoding,
                       const at::Tensor& out) {
    check_bf16_rows(q, "q", 3);
    check_bf16_rows(out, "out", 3);
    for (auto* t : {&slot_ids, &cached_lens, &num_decoding}) check_i32(*t, "index");
    DecodeCall d;
    d.c = cache_desc(k_cache, v_cache, k_scale, v_scale, k_calibration);
    d.B = (int32_t)q.size(0);
    d.hq = (int32_t)q.size(1);
    // kernels.py:292
    TORCH_CHECK(out.size(0) >= d.B && out.size(1) == d.hq && out.size(2) == q.size(2),
                "ie: out must be [>=B, Hq, D]");
    TORCH_CHECK(cached_lens.size(0) >= d.B && slot_ids.size(0) >= d.B,
                "ie: index tensors too short");
    d.ws_bytes = ie_decode_attention_workspace_size(d.B, d.hq, (int32_t)q.size(2));
    return d;
}

// The decode and prefill workspaces carry arrival counts that must be zero on entry and that
// every call leaves zero, so they are kept across calls: one per (device, stream, kind),
// allocated zeroed on first use and replaced by a larger one when a call needs more. Replaced
// buffers are kept too: a graph captured with one still addresses it. Calls in stream order
// never overlap on a buffer. Kinds: prefill; decode of up to 1024 sequences (their count
// regions coincide); decode of each larger batch size.
//
// Under hipGraph capture a call uses its stream's kept workspace when that stream has one (a
// warm-up on the capture stream made it, outside the capture: the pattern of GraphSet and
// DecodeStep). Otherwise (e.g. the engine's capture on torch's own capture stream after warming
// up on another, qwen3-1.7b/engine.py:432-449) the workspace is allocated inside the capture,
// from the graph's memory pool, and the graph records a fill of its count bytes before the
// first call that uses it, so every replay starts from zero counts whatever the pool put in
// that memory in between. Such a workspace serves the rest of the same capture; the reference
// to it is dropped when the stream starts its next capture (the graph keeps using the memory).
// A graph that uses a stream's kept workspace shares it with eager calls on that stream and
// with the other graphs captured there: replay those graphs one at a time and not beside eager
// calls on that stream, the rule torch already sets for graphs that share a memory pool.
constexpr int32_t WS_PREFILL = -1;
at::Tensor persistent_workspace(const at::Tensor& q, size_t bytes, size_t count_bytes,
                                int32_t kind) {
    using Key = std::tuple<int, hipStream_t, int32_t>;
    struct Captured {
        unsigned long long id = 0;
        std::map<int32_t, std::vector<at::Tensor>> held;
    };
    static std::mutex mu;
    static auto* eager = new std::map<Key, std::vector<at::Tensor>>();  // kept for the process
    static auto* captured = new std::map<std::pair<int, hipStream_t>, Captured>();
    const hipStream_t s = stream_of(q);
    const int dev = q.device().index();
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    ok(hipStreamGetCaptureInfo(s, &status, &id), "stream capture status");
    const int64_t n = (int64_t)std::max<size_t>(bytes, 256);
    std::lock_guard<std::mutex> lock(mu);
    auto& held = (*eager)[Key{dev, s, kind}];
    const bool fits = !held.empty() && held.back().numel() >= n;
    if (status == hipStreamCaptureStatusNone) {
        if (!fits) held.push_back(at::zeros({n}, q.options().dtype(at::kByte)));
        return held.back();
    }
    TORCH_CHECK(status == hipStreamCaptureStatusActive, "ie: the capture stream is invalidated");
    if (fits) return held.back();
    Captured& cap = (*captured)[{dev, s}];
    if (cap.id != id) {  // a new capture on this stream: the previous one has ended
        cap.id = id;
        cap.held.clear();
    }
    auto& mine = cap.held[kind];
    if (mine.empty() || mine.back().numel() < n) {
        at::Tensor w = at::empty({n}, q.options().dtype(at::kByte));
        w.narrow(0, 0, (int64_t)std::min<size_t>(count_bytes, (size_t)n)).zero_();  // recorded
        mine.push_back(w);
    }
    return mine.back();
}

void decode_attention(const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                      const at::Tensor& k_scale, const at::Tensor& v_scale,
                      const at::Tensor& k_calibration, const at::Tensor& cached_lens,
                      const at::Tensor& slot_ids, const at::Tensor& num_decoding, double scale,
                      const at::Tensor& out, const c10::optional<at::Tensor>& plan) {
    const c10::DeviceGuard guard(q.device());
    DecodeCall d = decode_prep(q, k_cache, v_cache, k_scale, v_scale, k_calibration, cached_lens,
                               slot_ids, num_decoding, out);
    at::Tensor ws = persistent_workspace(
        q, d.ws_bytes, ie_decode_attention_workspace_counts_bytes(d.B, d.hq),
        decode_ws_kind(d));
    if (plan.has_value()) {
        check_decode_plan(*plan, q);
        ok(ie_decode_attention_planned(bf(q), q.stride(0), q.stride(1), d.B, d.hq, &d.c,
                                       i32(cached_lens), i32(slot_ids), i32(num_decoding),
                                       i32(*plan), plan->size(0), (float)scale, bfm(out),
                                       out.stride(0), out.stride(1), ws.data_ptr(), d.ws_bytes,
                                       stream_of(q)),
           "decode_attention");
        return;
    }
    ok(ie_decode_attention(bf(q), q.stride(0), q.stride(1), d.B, d.hq, &d.c, i32(cached_lens),
                           i32(slot_ids), i32(num_decoding), (float)scale, bfm(out),
                           out.stride(0), out.stride(1), ws.data_ptr(), d.ws_bytes, stream_of(q)),
       "decode_attention");
}

// fused_rope_kv_decode then decode_attention in one launch (ie_decode_attention_rope): q, k, v
// are the QKV projection's raw rows.
void decode_attention_rope(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                           const at::Tensor& q_norm_weight, const at::Tensor& k_norm_weight,
                           const at::Tensor& cos, const at::Tensor& sin,
                           const at::Tensor& k_cache, const at::Tensor& v_cache,
                           const at::Tensor& k_scale, const at::Tensor& v_scale,
                           const at::Tensor& k_calibration, const at::Tensor& cached_lens,
                           const at::Tensor& slot_ids, const at::Tensor& num_decoding,
                           double eps, double scale, const at::Tensor& out,
                           const c10::optional<at::Tensor>& plan) {
    check_bf16_rows(k, "k", 3);
    check_bf16_rows(v, "v", 3);
    check_bf16_rows(q_norm_weight, "q_norm_weight", 1);
    check_bf16_rows(k_norm_weight, "k_norm_weight", 1);
    check_bf16_rows(cos, "cos", 3);
    check_bf16_rows(sin, "sin", 3);
    const c10::DeviceGuard guard(q.device());
    DecodeCall d = decode_prep(q, k_cache, v_cache, k_scale, v_scale, k_calibration, cached_lens,
                               slot_ids, num_decoding, out);
    TORCH_CHECK(q.size(2) == 128 && k.size(2) == 128 && v.size(2) == 128, "ie: head_dim 128");
    TORCH_CHECK(k.size(0) >= d.B && v.size(0) >= d.B && k.size(1) == d.c.num_kv_heads &&
                    v.size(1) == d.c.num_kv_heads,
                "ie: k/v shape mismatch");
    TORCH_CHECK(cos.size(0) >= d.B && sin.size(0) >= d.B && cos.size(2) == 64 && sin.size(2) == 64,
                "ie: cos/sin must be [B,1,64]");
    at::Tensor ws = persistent_workspace(
        q, d.ws_bytes, ie_decode_attention_workspace_counts_bytes(d.B, d.hq),
        decode_ws_kind(d));
    if (plan.has_value()) {
        check_decode_plan(*plan, q);
        ok(ie_decode_attention_rope_planned(
               bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1), bf(v),
               v.stride(0), v.stride(1), bf(q_norm_weight), bf(k_norm_weight), bf(cos),
               cos.stride(0), bf(sin), sin.stride(0), (float)eps, d.B, d.hq, &d.c,
               i32(cached_lens), i32(slot_ids), i32(num_decoding), i32(*plan), plan->size(0),
               (float)scale, bfm(out), out.stride(0), out.stride(1), ws.data_ptr(), d.ws_bytes,
               stream_of(q)),
           "decode_attention_rope");
        return;
    }
    ok(ie_decode_attention_rope(bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1),
                                bf(v), v.stride(0), v.stride(1), bf(q_norm_weight),
                                bf(k_norm_weight), bf(cos), cos.stride(0), bf(sin),
                                sin.stride(0), (float)eps, d.B, d.hq, &d.c, i32(cached_lens),
                                i32(slot_ids), i32(num_decoding), (float)scale, bfm(out),
                                out.stride(0), out.stride(1), ws.data_ptr(), d.ws_bytes,
                                stream_of(q)),
       "decode_attention_rope");
}

// The decode launch's work list for one step's metadata (ie_decode_attention_plan): int32
// [grid, 4] on cached_lens' device, to pass to every layer's decode launch of that step.
at::Tensor decode_plan(const at::Tensor& cached_lens, const at::Tensor& num_decoding,
                       int64_t batch, int64_t num_q_heads, int64_t num_kv_heads) {
    check_i32(cached_lens, "cached_lens");
    check_i32(num_decoding, "num_decoding");
    const c10::DeviceGuard guard(cached_lens.device());
    TORCH_CHECK(batch >= 0 && cached_lens.size(0) >= batch, "ie: cached_lens too short");
    TORCH_CHECK(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0 &&
                    num_q_heads / num_kv_heads <= 16,
                "ie: num_q_heads must be num_kv_heads times a GQA ratio of 1 to 16");
    const int32_t units =
        (int32_t)(num_kv_heads * ((num_q_heads / num_kv_heads + 1) / 2));
    const int32_t grid = ie_decode_attention_grid((int32_t)batch, units);
    at::Tensor rows = at::empty({std::max(grid, 1), 4}, cached_lens.options());
    ok(ie_decode_attention_plan(i32(cached_lens), i32(num_decoding), (int32_t)batch, units,
                                i32m(rows), stream_of(cached_lens)),
       "decode_plan");
    return rows;
}

// The LM head and greedy sampling in one launch (ie_skinny_lm_head_greedy): h [M, K] (the
// residual stream with norm, else the normed rows), weight swizzled for n_tiles; returns
// (logits [M, N], tokens [M, 1] int64) and advances seed by one, as sample does at tau 0.
constexpr int32_t WS_LM_HEAD = -2;
std::tuple<at::Tensor, at::Tensor> lm_head_greedy(const at::Tensor& h, const at::Tensor& weight,
                                                  int64_t n_tiles, double eps, bool norm,
                                                  const at::Tensor& seed) {
    check_bf16_rows(h, "h", 2);
    check_bf16_rows(weight, "weight", 2);
    TORCH_CHECK(seed.is_cuda() && seed.scalar_type() == at::kLong && seed.numel() >= 1 &&
                    seed.is_contiguous() && seed.device() == h.device() &&
                    weight.device() == h.device(),
                "ie: seed must be an int64 tensor on h's device, with the weight");
    const c10::DeviceGuard guard(h.device());
    const int64_t M = h.size(0), K = h.size(1), N = weight.size(0);
    TORCH_CHECK(weight.size(1) == K && weight.is_contiguous(), "ie: weight must be [N, K]");
    at::Tensor logits = at::empty({M, N}, h.options());
    at::Tensor tokens = at::empty({M, 1}, h.options().dtype(at::kLong));
    const size_t wsb = ie_skinny_lm_head_greedy_workspace_size();
    at::Tensor ws = persistent_workspace(h, wsb, wsb, WS_LM_HEAD);
    ok(ie_skinny_lm_head_greedy(bf(h), h.stride(0), (int32_t)M, bf(weight), (int32_t)N,
                                (int32_t)K, (int32_t)n_tiles, norm ? IE_SKINNY_NORM : 0,
                                (float)eps, bfm(logits), logits.stride(0),
                                tokens.data_ptr<int64_t>(), tokens.stride(0),
                                seed.data_ptr<int64_t>(), ws.data_ptr(), wsb, stream_of(h)),
       "lm_head_greedy");
    return {logits, tokens};
}

// A decode step's per-step inputs in one launch (ie_decode_step_prologue): the embedding rows
// of ids, the decode work list (as decode_plan) and the RoPE tables of positions cached_lens
// (as rope_tables). Returns (x [B, D], plan, cos [B, 1, H], sin).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> decode_step_prologue(
    const at::Tensor& ids, const at::Tensor& embed, const at::Tensor& cached_lens,
    const at::Tensor& num_decoding, int64_t num_q_heads, int64_t num_kv_heads,
    const at::Tensor& inv_freq) {
    check_i32(cached_lens, "cached_lens");
    check_i32(num_decoding, "num_decoding");
    check_bf16_rows(embed, "embed", 2);
    check_dev(ids, "ids");
    check_dev(inv_freq, "inv_freq");
    TORCH_CHECK(ids.scalar_type() == at::kLong && ids.is_contiguous() &&
                    ids.device() == cached_lens.device() && embed.device() == ids.device(),
                "ie: ids must be contiguous int64 on the device of cached_lens and embed");
    TORCH_CHECK(inv_freq.scalar_type() == at::kFloat && inv_freq.dim() == 1 &&
                    inv_freq.is_contiguous() && inv_freq.device() == cached_lens.device(),
                "ie: inv_freq must be a contiguous fp32 vector on the cached_lens' device");
    TORCH_CHECK(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0 &&
                    num_q_heads / num_kv_heads <= 16,
                "ie: num_q_heads must be num_kv_heads times a GQA ratio of 1 to 16");
    const c10::DeviceGuard guard(cached_lens.device());
    const int64_t B = ids.numel(), D = embed.size(1), H = inv_freq.size(0);
    TORCH_CHECK(cached_lens.size(0) >= B, "ie: cached_lens too short");
    const int32_t units =
        (int32_t)(num_kv_heads * ((num_q_heads / num_kv_heads + 1) / 2));
    const int32_t grid = ie_decode_attention_grid((int32_t)B, units);
    at::Tensor rows = at::empty({std::max(grid, 1), 4}, cached_lens.options());
    auto bopt = embed.options();
    at::Tensor x = at::empty({B, D}, bopt), c = at::empty({B, 1, H}, bopt),
               s = at::empty({B, 1, H}, bopt);
    ok(ie_decode_step_prologue(i32(cached_lens), i32(num_decoding), (int32_t)B, units,
                               i32m(rows), inv_freq.data_ptr<float>(), (int32_t)H, bfm(c),
                               bfm(s), ids.data_ptr<int64_t>(), bf(embed), embed.stride(0),
                               embed.size(0), (int32_t)D, bfm(x), x.stride(0),
                               stream_of(cached_lens)),
       "decode_step_prologue");
    return {x, rows, c, s};
}

int64_t decode_attention_workspace_size(int64_t batch, int64_t num_q_heads) {
    return (int64_t)ie_decode_attention_workspace_size((int32_t)batch, (int32_t)num_q_heads, 128);
}

void dequantize_kv_prefix(const at::Tensor& k_cache, const at::Tensor& v_cache,
                          const at::Tensor& k_scale, const at::Tensor& v_scale,
                          const at::Tensor& k_calibration, const at::Tensor& cu_cached,
                          const at::Tensor& slot_ids, const at::Tensor& k_out,
                          const at::Tensor& v_out) {
    check_i32(cu_cached, "cu_cached");
    check_i32(slot_ids, "slot_ids");
    check_bf16_rows(k_out, "k_out", 3);
    check_bf16_rows(v_out, "v_out", 3);
    TORCH_CHECK(k_out.strides() == v_out.strides(), "ie: k_out/v_out strides differ");
    const c10::DeviceGuard guard(k_cache.device());
    ie_kv_cache c = cache_desc(k_cache, v_cache, k_scale, v_scale, k_calibration);
    const int32_t entries = (int32_t)cu_cached.size(0) - 1;
    ok(ie_dequantize_kv_prefix(&c, i32(cu_cached), i32(slot_ids), entries, bfm(k_out), bfm(v_out),
                               k_out.stride(0), k_out.stride(1), stream_of(k_cache)),
       "dequantize_kv_prefix");
}

at::Tensor prefill_attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             const at::Tensor& seq_ids, const at::Tensor& cu_seqlens,
                             const at::Tensor& tile_start, const at::Tensor& k_cache,
                             const at::Tensor& v_cache, const at::Tensor& k_scale,
                             const at::Tensor& v_scale, const at::Tensor& k_calibration,
                             const at::Tensor& slot_ids, const at::Tensor& cu_cached,
                             int64_t block_m, const c10::optional<at::Tensor>& plan) {
    check_bf16_rows(q, "q", 3);
    check_bf16_rows(k, "k", 3);
    check_bf16_rows(v, "v", 3);
    for (auto* t : {&seq_ids, &cu_seqlens, &tile_start, &slot_ids, &cu_cached})
        check_i32(*t, "index");
    const c10::DeviceGuard guard(q.device());
    ie_kv_cache c = cache_desc(k_cache, v_cache, k_scale, v_scale, k_calibration);
    const int64_t N = q.size(0);
    TORCH_CHECK(k.size(0) == N && v.size(0) == N && k.size(1) == c.num_kv_heads &&
                    v.size(1) == c.num_kv_heads,
                "ie: k/v shape mismatch");
    // the kernel reads cu_seqlens/cu_cached[0 .. entries] and seq_ids[0 .. N) on the device
    TORCH_CHECK(slot_ids.size(0) >= 1 && cu_seqlens.size(0) == slot_ids.size(0) + 1 &&
                    cu_cached.size(0) == slot_ids.size(0) + 1,
                "ie: cu_seqlens and cu_cached must hold len(slot_ids) + 1 entries");
    TORCH_CHECK(seq_ids.size(0) >= N, "ie: seq_ids must hold one entry per packed row");
    at::Tensor out = at::empty({N, q.size(1), q.size(2)}, q.options());
    const size_t ws_bytes = ie_prefill_attention_workspace_size(
        (int32_t)tile_start.size(0), (int32_t)block_m, c.num_kv_heads);
    at::Tensor ws = persistent_workspace(q, ws_bytes,
                                         ie_prefill_attention_workspace_counts_bytes(), WS_PREFILL);
    if (plan.has_value()) {
        const at::Tensor& p = *plan;
        check_dev(p, "plan");
        TORCH_CHECK(p.scalar_type() == at::kInt && p.dim() == 2 && p.size(1) == 16 &&
                        p.is_contiguous(),
                    "ie: plan must be the [grid, 16] int32 tensor prefill_plan returns");
        ok(ie_prefill_attention_planned(
               bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1), bf(v),
               v.stride(0), v.stride(1), N, (int32_t)q.size(1), i32(seq_ids), i32(cu_seqlens),
               i32(tile_start), (int32_t)tile_start.size(0), (int32_t)block_m, &c, i32(slot_ids),
               i32(cu_cached), (int32_t)slot_ids.size(0), i32(p), p.size(0), bfm(out),
               out.stride(0), out.stride(1), ws.data_ptr(), ws_bytes, stream_of(q)),
           "prefill_attention (planned)");
        return out;
    }
    ok(ie_prefill_attention(bf(q), q.stride(0), q.stride(1), bf(k), k.stride(0), k.stride(1),
                            bf(v), v.stride(0), v.stride(1), N, (int32_t)q.size(1), i32(seq_ids),
                            i32(cu_seqlens), i32(tile_start), (int32_t)tile_start.size(0),
                            (int32_t)block_m, &c, i32(slot_ids), i32(cu_cached),
                            (int32_t)slot_ids.size(0), bfm(out),
                            out.stride(0), out.stride(1), ws.data_ptr(), ws_bytes, stream_of(q)),
       "prefill_attention");
    return out;
}

// The prefill launch's work list for one step's metadata (see ie_prefill_attention_plan):
// [grid, 16] int32 on the metadata's device, to pass to every layer's prefill_attention.
at::Tensor prefill_plan(const at::Tensor& seq_ids, const at::Tensor& cu_seqlens,
                        const at::Tensor& tile_start, const at::Tensor& slot_ids,
                        const at::Tensor& cu_cached, int64_t num_tokens, int64_t num_q_heads,
                        int64_t num_kv_heads, int64_t block_m) {
    for (auto* t : {&seq_ids, &cu_seqlens, &tile_start, &slot_ids, &cu_cached})
        check_i32(*t, "index");
    const c10::DeviceGuard guard(seq_ids.device());
    TORCH_CHECK(slot_ids.size(0) >= 1 && cu_seqlens.size(0) == slot_ids.size(0) + 1 &&
                    cu_cached.size(0) == slot_ids.size(0) + 1,
                "ie: cu_seqlens and cu_cached must hold len(slot_ids) + 1 entries");
    TORCH_CHECK(seq_ids.size(0) >= num_tokens, "ie: seq_ids must hold one entry per packed row");
    const int32_t nt = (int32_t)tile_start.size(0);
    const int32_t grid = ie_prefill_attention_grid(nt, (int32_t)block_m, (int32_t)num_q_heads,
                                                   (int32_t)num_kv_heads);
    // the plan kernel writes every row of a launch (a workgroup without work: zeros)
    at::Tensor rows = grid > 0 ? at::empty({grid, 16}, seq_ids.options())
                               : at::zeros({1, 16}, seq_ids.options());
    ok(ie_prefill_attention_plan(i32(seq_ids), i32(cu_seqlens), i32(tile_start), nt,
                                 (int32_t)block_m, num_tokens, (int32_t)num_q_heads,
                                 (int32_t)num_kv_heads, i32(slot_ids), i32(cu_cached),
                                 (int32_t)slot_ids.size(0), i32m(rows), stream_of(seq_ids)),
       "prefill_plan");
    return rows;
}

}  // namespace

TORCH_LIBRARY(ie, m) {
    m.def(
        "quantize_kv_prefill(Tensor k, Tensor v, Tensor cu_seqlens, Tensor slot_ids, "
        "Tensor cached_lens, Tensor num_decoding, Tensor(a!) k_cache, Tensor(b!) v_cache, "
        "Tensor(c!) k_scale, Tensor(d!) v_scale, Tensor(e!) k_calibration) -> ()");
    m.def(
        "fused_rope_kv_decode(Tensor q, Tensor k, Tensor v, Tensor q_norm_weight, "
        "Tensor k_norm_weight, Tensor cos, Tensor sin, Tensor slot_ids, Tensor(a!) k_cache, "
        "Tensor(b!) v_cache, Tensor(c!) k_scale, Tensor(d!) v_scale, Tensor k_calibration, "
        "Tensor cached_lens, Tensor num_decoding, float eps) -> Tensor");
    m.def(
        "fused_norm_rope_prefill(Tensor q, Tensor k, Tensor q_norm_weight, Tensor k_norm_weight, "
        "Tensor cos, Tensor sin, float eps) -> (Tensor, Tensor)");
    m.def("sample(Tensor logits, float tau, Tensor(a!) seed) -> Tensor");
    m.def("add_rms_norm(Tensor residual, Tensor delta, Tensor weight, float eps) -> (Tensor, Tensor)");
    m.def("silu_mul(Tensor gate_up) -> Tensor");
    m.def("rope_tables(Tensor positions, Tensor inv_freq) -> (Tensor, Tensor)");
    m.def("skinny_matmul(Tensor x, Tensor weight, int n_tiles=1, bool swizzled=False) -> Tensor");
    m.def(
        "skinny_matmul_silu_mul(Tensor x, Tensor weight, int n_tiles=1, bool swizzled=False) "
        "-> Tensor");
    m.def(
        "skinny_matmul_norm(Tensor h, Tensor weight, int n_tiles, bool silu_mul, float eps, "
        "bool swizzled=False, bool fragments=False) -> Tensor");
    m.def(
        "skinny_matmul_residual_(Tensor x, Tensor weight, int n_tiles, Tensor(a!) residual, "
        "bool swizzled=False, bool x_fragments=False) -> Tensor(a!)");
    m.def("skinny_weight_swizzle(Tensor weight, int n_tiles, bool gate_up=False) -> Tensor");
    m.def(
        "decode_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor k_scale, "
        "Tensor v_scale, Tensor k_calibration, Tensor cached_lens, Tensor slot_ids, "
        "Tensor num_decoding, float scale, Tensor(a!) out, Tensor? plan=None) -> ()");
    m.def(
        "decode_attention_rope(Tensor q, Tensor k, Tensor v, Tensor q_norm_weight, "
        "Tensor k_norm_weight, Tensor cos, Tensor sin, Tensor(a!) k_cache, Tensor(b!) v_cache, "
        "Tensor(c!) k_scale, Tensor(d!) v_scale, Tensor k_calibration, Tensor cached_lens, "
        "Tensor slot_ids, Tensor num_decoding, float eps, float scale, Tensor(e!) out, "
        "Tensor? plan=None) -> ()");
    m.def(
        "decode_plan(Tensor cached_lens, Tensor num_decoding, int batch, int num_q_heads, "
        "int num_kv_heads) -> Tensor");
    m.def(
        "lm_head_greedy(Tensor h, Tensor weight, int n_tiles, float eps, bool norm, "
        "Tensor(a!) seed) -> (Tensor, Tensor)");
    m.def(
        "decode_step_prologue(Tensor ids, Tensor embed, Tensor cached_lens, Tensor num_decoding, "
        "int num_q_heads, int num_kv_heads, Tensor inv_freq) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("decode_attention_workspace_size(int batch, int num_q_heads) -> int");
    m.def(
        "dequantize_kv_prefix(Tensor k_cache, Tensor v_cache, Tensor k_scale, Tensor v_scale, "
        "Tensor k_calibration, Tensor cu_cached, Tensor slot_ids, Tensor(a!) k_out, "
        "Tensor(b!) v_out) -> ()");
    m.def(
        "prefill_attention(Tensor q, Tensor k, Tensor v, Tensor seq_ids, Tensor cu_seqlens, "
        "Tensor tile_start, Tensor k_cache, Tensor v_cache, Tensor k_scale, Tensor v_scale, "
        "Tensor k_calibration, Tensor slot_ids, Tensor cu_cached, int block_m, "
        "Tensor? plan=None) -> Tensor");
    m.def(
        "prefill_plan(Tensor seq_ids, Tensor cu_seqlens, Tensor tile_start, Tensor slot_ids, "
        "Tensor cu_cached, int num_tokens, int num_q_heads, int num_kv_heads, int block_m) "
        "-> Tensor");
    m.impl("decode_attention_workspace_size", &decode_attention_workspace_size);
}

TORCH_LIBRARY_IMPL(ie, CUDA, m) {
    m.impl("quantize_kv_prefill", &quantize_kv_prefill);
    m.impl("fused_rope_kv_decode", &fused_rope_kv_decode);
    m.impl("fused_norm_rope_prefill", &fused_norm_rope_prefill);
    m.impl("sample", &sample);
    m.impl("add_rms_norm", &add_rms_norm);
    m.impl("silu_mul", &silu_mul);
    m.impl("rope_tables", &rope_tables);
    m.impl("skinny_matmul", &skinny_matmul);
    m.impl("skinny_matmul_silu_mul", &skinny_matmul_silu_mul);
    m.impl("skinny_matmul_norm", &skinny_matmul_norm);
    m.impl("skinny_matmul_residual_", &skinny_matmul_residual_);
    m.impl("decode_step_prologue", &decode_step_prologue);
    m.impl("lm_head_greedy", &lm_head_greedy);
    m.impl("skinny_weight_swizzle", &skinny_weight_swizzle);
    m.impl("decode_attention", &decode_attention);
    m.impl("decode_attention_rope", &decode_attention_rope);
    m.impl("dequantize_kv_prefix", &dequantize_kv_prefix);
    m.impl("prefill_attention", &prefill_attention);
    m.impl("prefill_plan", &prefill_plan);
    m.impl("decode_plan", &decode_plan);
}
