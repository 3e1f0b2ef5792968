// Per-layer residual add + RMSNorm and SiLU-gated product (gfx950), the elementwise steps between
// the projections of a Qwen3 block (qwen3-1.7b/kernels.py:1178-1283, called at
// architecture.py:224,282,300,412).
//
// add_rms_norm_kernel, grid N, 256 threads: one token row. Thread t owns elements
// 8t + 2048j + i (16-byte loads of 8 bf16); the new residual bf16(residual + delta) stays in
// registers for the norm. Sum of squares in a fixed order: each thread adds its squares in
// element order, the wave combines by the xor butterfly, the four wave sums are added in wave
// order; rstd = 1 / sqrt(ss / D + eps) (IEEE); normed = bf16((r * rstd) * w).
// silu_mul_kernel, grid (N, cdiv(D, 2048)), 256 threads x 8 elements: bf16((g * sigmoid(g)) * u).
// Both are HBM-bound streams (each byte read or written once).
// rope_tables_kernel: the RoPE cos/sin tables of a step's positions (architecture.py:382-390) in
// one launch instead of PyTorch's five elementwise ones.
#include "ie_common.h"

namespace ie {

constexpr int NA_THREADS = 256;
constexpr int NA_VEC = 8;
constexpr int NA_STEP = NA_THREADS * NA_VEC;  // 2048 elements per pass
constexpr int NA_MAX_PASSES = 4;              // D <= 8192

__device__ __forceinline__ void unpack8(uint4 w, float (&x)[NA_VEC]) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = bf16lo(ws[j]);
        x[2 * j + 1] = bf16hi(ws[j]);
    }
}
__device__ __forceinline__ uint4 pack8(const float (&x)[NA_VEC]) {
    return make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                      pack_bf16x2(x[6], x[7]));
}

__global__ __launch_bounds__(NA_THREADS) void add_rms_norm_kernel(
    const uint16_t* __restrict__ res, int64_t rs, const uint16_t* __restrict__ delta, int64_t ds,
    const uint16_t* __restrict__ w, int D, float eps, uint16_t* __restrict__ nres, int64_t nrs,
    uint16_t* __restrict__ normed, int64_t ns) {
#pragma clang fp contract(off)
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x;
    const int passes = (D + NA_STEP - 1) / NA_STEP;
    float r[NA_MAX_PASSES][NA_VEC];
    uint4 wraw[NA_MAX_PASSES];  // the weight, loaded with the row (not after the reduction)
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NA_MAX_PASSES; ++j) {
        const int c = j * NA_STEP + NA_VEC * tid;
        if (j < passes && c < D) wraw[j] = *reinterpret_cast<const uint4*>(w + c);
    }
#pragma unroll
    for (int j = 0; j < NA_MAX_PASSES; ++j) {
        const int c = j * NA_STEP + NA_VEC * tid;
        if (j < passes && c < D) {
            float a[NA_VEC], b[NA_VEC];
            unpack8(*reinterpret_cast<const uint4*>(res + t * rs + c), a);
            unpack8(*reinterpret_cast<const uint4*>(delta + t * ds + c), b);
#pragma unroll
            for (int i = 0; i < NA_VEC; ++i) r[j][i] = bf16_to_f32(f32_to_bf16_rne(a[i] + b[i]));
            *reinterpret_cast<uint4*>(nres + t * nrs + c) = pack8(r[j]);
#pragma unroll
            for (int i = 0; i < NA_VEC; ++i) acc = acc + r[j][i] * r[j][i];
        }
    }
    acc = wave_sum_butterfly(acc);
    __shared__ float s_w[NA_THREADS / IE_WAVE];
    if ((tid & 63) == 0) s_w[tid >> 6] = acc;
    __syncthreads();
    float ss = s_w[0];
#pragma unroll
    for (int i = 1; i < NA_THREADS / IE_WAVE; ++i) ss = ss + s_w[i];
    const float rstd = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < NA_MAX_PASSES; ++j) {
        const int c = j * NA_STEP + NA_VEC * tid;
        if (j < passes && c < D) {
            float wv[NA_VEC], y[NA_VEC];
            unpack8(wraw[j], wv);
#pragma unroll
            for (int i = 0; i < NA_VEC; ++i) y[i] = (r[j][i] * rstd) * wv[i];
            *reinterpret_cast<uint4*>(normed + t * ns + c) = pack8(y);
        }
    }
}

__global__ __launch_bounds__(NA_THREADS) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                              int64_t gs, int D,
                                                              uint16_t* __restrict__ out,
                                                              int64_t os) {
#pragma clang fp contract(off)
    const int64_t t = blockIdx.x;
    const int c = blockIdx.y * NA_STEP + NA_VEC * threadIdx.x;
    if (c >= D) return;
    float g[NA_VEC], u[NA_VEC], y[NA_VEC];
    unpack8(*reinterpret_cast<const uint4*>(gu + t * gs + c), g);
    unpack8(*reinterpret_cast<const uint4*>(gu + t * gs + D + c), u);
#pragma unroll
    for (int i = 0; i < NA_VEC; ++i) {
        const float s = 1.0f / (1.0f + expf(-g[i]));
        y[i] = (g[i] * s) * u[i];
    }
    *reinterpret_cast<uint4*>(out + t * os + c) = pack8(y);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace ie

using namespace ie;

extern "C" hipError_t ie_add_rms_norm(const ie_bf16* residual, int64_t residual_stride,
                                      const ie_bf16* delta, int64_t delta_stride,
                                      const ie_bf16* weight, int64_t num_tokens, int32_t dim,
                                      float eps, ie_bf16* new_residual,
                                      int64_t new_residual_stride, ie_bf16* normed,
                                      int64_t normed_stride, hipStream_t stream) {
    IE_REQUIRE(num_tokens >= 0 && dim > 0, "bad sizes");
    if (num_tokens == 0) return hipSuccess;
    IE_REQUIRE(residual && delta && weight && new_residual && normed, "null pointer");
    IE_REQUIRE(dim % NA_VEC == 0 && dim <= NA_STEP * NA_MAX_PASSES,
               "dim must be a multiple of 8, at most 8192");
    IE_REQUIRE(aligned16(residual) && aligned16(delta) && aligned16(weight) &&
                   aligned16(new_residual) && aligned16(normed) && residual_stride % 8 == 0 &&
                   delta_stride % 8 == 0 && new_residual_stride % 8 == 0 && normed_stride % 8 == 0,
               "rows must be 16-byte aligned");
    IE_REQUIRE(num_tokens < (1LL << 31), "too many tokens");
    hipLaunchKernelGGL(add_rms_norm_kernel, dim3((unsigned)num_tokens), dim3(NA_THREADS), 0,
                       stream, (const uint16_t*)residual, residual_stride,
                       (const uint16_t*)delta, delta_stride, (const uint16_t*)weight, dim, eps,
                       (uint16_t*)new_residual, new_residual_stride, (uint16_t*)normed,
                       normed_stride);
    return hipGetLastError();
}

extern "C" hipError_t ie_silu_mul(const ie_bf16* gate_up, int64_t gate_up_stride,
                                  int64_t num_tokens, int32_t dim, ie_bf16* out,
                                  int64_t out_stride, hipStream_t stream) {
    IE_REQUIRE(num_tokens >= 0 && dim > 0, "bad sizes");
    if (num_tokens == 0) return hipSuccess;
    IE_REQUIRE(gate_up && out, "null pointer");
    IE_REQUIRE(dim % NA_VEC == 0, "dim must be a multiple of 8");
    IE_REQUIRE(aligned16(gate_up) && aligned16(out) && gate_up_stride % 8 == 0 &&
                   out_stride % 8 == 0,
               "rows must be 16-byte aligned");
    IE_REQUIRE(num_tokens < (1LL << 31), "too many tokens");
    dim3 grid((unsigned)num_tokens, (unsigned)((dim + NA_STEP - 1) / NA_STEP));
    hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(NA_THREADS), 0, stream,
                       (const uint16_t*)gate_up, gate_up_stride, dim, (uint16_t*)out, out_stride);
    return hipGetLastError();
}

namespace ie {

// angle = float(position) * inv_freq[j] (one IEEE fp32 product), then cos and sin of it (the
// device library's cosf/sinf) rounded to bf16: the arithmetic of the reference's
// `positions[:, None, None] * inv_freq` then `.cos().to(bf16)`, `.sin().to(bf16)`.
__global__ __launch_bounds__(256) void rope_tables_kernel(const int32_t* __restrict__ pos,
                                                          int64_t n, const float* __restrict__ inv,
                                                          int half, uint16_t* __restrict__ cosv,
                                                          uint16_t* __restrict__ sinv) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n * half) return;
    rope_table_entry(pos, inv, i, half, cosv, sinv);
}

}  // namespace ie

extern "C" hipError_t ie_rope_tables(const int32_t* positions, int64_t n, const float* inv_freq,
                                     int32_t half_dim, ie_bf16* cos_out, ie_bf16* sin_out,
                                     hipStream_t stream) {
    IE_REQUIRE(n >= 0 && half_dim > 0, "bad sizes");
    if (n == 0) return hipSuccess;
    IE_REQUIRE(positions && inv_freq && cos_out && sin_out, "null pointer");
    const int64_t total = n * half_dim;
    IE_REQUIRE(total / 256 < (1LL << 31), "too many table entries");
    hipLaunchKernelGGL(ie::rope_tables_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, positions, n, inv_freq, (int)half_dim, (uint16_t*)cos_out,
                       (uint16_t*)sin_out);
    return hipGetLastError();
}
