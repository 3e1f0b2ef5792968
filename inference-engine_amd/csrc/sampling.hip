// Token sampling over the vocabulary (gfx950): Gumbel-max with Triton's Philox uniforms, greedy
// argmax at tau = 0.
//
// Semantics (qwen3-1.7b/kernels.py:1286-1370): token[b] = the first v maximizing
// logits[b, v] + tau * -log(-log(clamp(u[b, v], 1e-10, 1 - 1e-7))), u = tl.rand(seed, b * V + v):
// Philox4x32-10 on counter (b * V + v as int32, 0, 0, 0) and key (seed low word, seed high word),
// first output word x as int32, u = float(x < 0 ? -x - 1 : x) * 4.6566127342e-10. Then the
// device seed is incremented. At tau = 0 the noise term is 0 * finite, so no uniform is drawn.
//
// Two launches, HBM-bound at tau = 0 (B x V logits read once): sample_partial_kernel, grid
// (cdiv(V, 8192), B), 256 threads x 32 entries (16-byte loads) -> the best (value, index) of each
// block of 8192 entries; sample_combine_kernel, grid B, one wave: the best over the row's blocks,
// and the seed increment (after every block has read the seed: the launches are stream-ordered).
#include "ie_common.h"

namespace ie {

constexpr int SP_THREADS = 256;
constexpr int SP_VEC = 8;                                // entries per 16-byte bf16 load
constexpr int SP_ROUNDS = 4;                             // loads per thread
constexpr int SP_BLOCK = SP_THREADS * SP_VEC * SP_ROUNDS;  // 8192 entries per workgroup

struct Best {
    float v;
    int i;
};
// (a, b) ordered as the reference's argmax: larger value, then smaller index
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}
__device__ __forceinline__ void take(Best& best, float v, int i) {
    if (better(v, i, best.v, best.i)) {
        best.v = v;
        best.i = i;
    }
}
__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(b.v, m, IE_WAVE);
        const int oi = __shfl_xor(b.i, m, IE_WAVE);
        take(b, ov, oi);
    }
    return b;
}

// Philox4x32-10, first output word, for counter (c0, 0, 0, 0) and key (k0, k1).
__device__ __forceinline__ uint32_t philox_first(uint32_t c0, uint32_t k0, uint32_t k1) {
    uint32_t c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t h0 = __umulhi(0xD2511F53u, c0), l0 = 0xD2511F53u * c0;
        const uint32_t h1 = __umulhi(0xCD9E8D57u, c2), l1 = 0xCD9E8D57u * c2;
        c0 = h1 ^ c1 ^ k0;
        c1 = l1;
        c2 = h0 ^ c3 ^ k1;
        c3 = l0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// The Gumbel-perturbed logit of entry `offset` (b * V + v, int32 arithmetic as the reference).
__device__ __forceinline__ float gumbel(float x, float tau, uint32_t offset, uint32_t k0,
                                        uint32_t k1) {
#pragma clang fp contract(off)
    const int32_t w = (int32_t)philox_first(offset, k0, k1);
    const float u0 = (float)(w ^ (w >> 31)) * 4.6566127342e-10f;  // x < 0 ? -x - 1 : x
    const float u = fminf(fmaxf(u0, 1e-10f), 0.99999988f);        // clamp(u, 1e-10, 1 - 1e-7)
    const float g = -logf(-logf(u));
    return x + tau * g;
}

template <typename T>
__device__ __forceinline__ void load8(const T* row, int64_t v, float (&x)[SP_VEC]);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* row, int64_t v, float (&x)[SP_VEC]) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + v);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = bf16lo(ws[j]);
        x[2 * j + 1] = bf16hi(ws[j]);
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float* row, int64_t v, float (&x)[SP_VEC]) {
    const float4 a = *reinterpret_cast<const float4*>(row + v);
    const float4 b = *reinterpret_cast<const float4*>(row + v + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// grid (cdiv(V, 8192), B), block 256: the best (value, index) of entries [8192 bx, +8192) of
// row by, to partial slot by * gridDim.x + bx. `vec_ok`: V is a multiple of 8 and the row start
// 16-byte aligned, so whole 8-entry groups load at once; otherwise entry by entry.
template <typename T>
__global__ __launch_bounds__(SP_THREADS) void sample_partial_kernel(
    const T* __restrict__ logits, int64_t ls, int64_t V, float tau,
    const int64_t* __restrict__ seed, int vec_ok, float* __restrict__ pv, int* __restrict__ pi) {
    const int b = blockIdx.y;
    const T* row = logits + b * ls;
    const int64_t base = (int64_t)blockIdx.x * SP_BLOCK;
    const int tid = threadIdx.x;
    const uint64_t sd = (uint64_t)seed[0];
    const uint32_t k0 = (uint32_t)sd, k1 = (uint32_t)(sd >> 32);
    const uint32_t row_off = (uint32_t)b * (uint32_t)V;
    Best best = {-INFINITY, 0x7fffffff};
    float x[SP_ROUNDS][SP_VEC];
#pragma unroll
    for (int r = 0; r < SP_ROUNDS; ++r) {
        const int64_t v0 = base + (int64_t)(r * SP_THREADS + tid) * SP_VEC;
        if (vec_ok && v0 + SP_VEC <= V) {
            load8<T>(row, v0, x[r]);
        } else {
#pragma unroll
            for (int j = 0; j < SP_VEC; ++j) {
                float y = -INFINITY;
                if (v0 + j < V) {
                    if constexpr (sizeof(T) == 2) y = bf16_to_f32(row[v0 + j]);
                    else y = (float)row[v0 + j];
                }
                x[r][j] = y;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < SP_ROUNDS; ++r) {
        const int64_t v0 = base + (int64_t)(r * SP_THREADS + tid) * SP_VEC;
#pragma unroll
        for (int j = 0; j < SP_VEC; ++j) {
            const int64_t v = v0 + j;
            if (v >= V) continue;
            float y = x[r][j];
            if (tau != 0.f) y = gumbel(y, tau, row_off + (uint32_t)v, k0, k1);
            take(best, y, (int)v);
        }
    }
    best = wave_best(best);
    __shared__ float s_v[SP_THREADS / IE_WAVE];
    __shared__ int s_i[SP_THREADS / IE_WAVE];
    if ((tid & 63) == 0) {
        s_v[tid >> 6] = best.v;
        s_i[tid >> 6] = best.i;
    }
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 1; w < SP_THREADS / IE_WAVE; ++w) take(best, s_v[w], s_i[w]);
        pv[b * gridDim.x + blockIdx.x] = best.v;
        pi[b * gridDim.x + blockIdx.x] = best.i;
    }
}

// grid max(B, 1), block 64: token of row b = the best of its nblk partials; workgroup 0 also
// advances the seed.
__global__ __launch_bounds__(64) void sample_combine_kernel(const float* __restrict__ pv,
                                                           const int* __restrict__ pi, int nblk,
                                                           int B, int64_t* __restrict__ out,
                                                           int64_t os, int64_t* __restrict__ seed) {
    const int b = blockIdx.x, lane = threadIdx.x;
    if (b < B) {
        Best best = {-INFINITY, 0x7fffffff};
        for (int j = lane; j < nblk; j += IE_WAVE) take(best, pv[b * nblk + j], pi[b * nblk + j]);
        best = wave_best(best);
        if (lane == 0) out[b * os] = best.i;
    }
    if (b == 0 && lane == 0) seed[0] += 1;
}

}  // namespace ie

using namespace ie;

extern "C" size_t ie_sample_workspace_size(int32_t batch, int64_t vocab) {
    if (batch <= 0 || vocab <= 0) return 0;
    const int64_t nblk = (vocab + SP_BLOCK - 1) / SP_BLOCK;
    return (size_t)batch * (size_t)nblk * (sizeof(float) + sizeof(int));
}

extern "C" hipError_t ie_sample(const void* logits, int32_t logits_dtype, int64_t logits_stride_row,
                                int32_t batch, int64_t vocab, float tau, int64_t* seed,
                                int64_t* out, int64_t out_stride_row, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
    IE_REQUIRE(batch >= 0 && vocab >= 0, "negative sizes");
    IE_REQUIRE(seed, "null pointer");
    IE_REQUIRE(logits_dtype == IE_DTYPE_BF16 || logits_dtype == IE_DTYPE_F32,
               "logits must be bf16 or fp32");
    IE_REQUIRE(vocab < (1LL << 31), "vocab must fit int32 indices");
    IE_REQUIRE(batch == 0 || vocab > 0, "empty vocabulary");
    const int64_t nblk = (vocab + SP_BLOCK - 1) / SP_BLOCK;
    float* pv = nullptr;
    int* pi = nullptr;
    if (batch > 0) {
        IE_REQUIRE(logits && out && workspace, "null pointer");
        IE_REQUIRE(workspace_bytes >= ie_sample_workspace_size(batch, vocab), "workspace too small");
        IE_REQUIRE(nblk < 65536, "vocab too large");
        pv = reinterpret_cast<float*>(workspace);
        pi = reinterpret_cast<int*>(pv + (size_t)batch * nblk);
        const size_t esz = logits_dtype == IE_DTYPE_BF16 ? 2 : 4;
        const int vec_ok = vocab % SP_VEC == 0 && (logits_stride_row * (int64_t)esz) % 16 == 0 &&
                           (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
        dim3 grid((unsigned)nblk, (unsigned)batch);
        if (logits_dtype == IE_DTYPE_BF16)
            hipLaunchKernelGGL(sample_partial_kernel<uint16_t>, grid, dim3(SP_THREADS), 0, stream,
                               (const uint16_t*)logits, logits_stride_row, vocab, tau,
                               (const int64_t*)seed, vec_ok, pv, pi);
        else
            hipLaunchKernelGGL(sample_partial_kernel<float>, grid, dim3(SP_THREADS), 0, stream,
                               (const float*)logits, logits_stride_row, vocab, tau,
                               (const int64_t*)seed, vec_ok, pv, pi);
    }
    hipLaunchKernelGGL(sample_combine_kernel, dim3((unsigned)std::max(batch, 1)), dim3(64), 0,
                       stream, pv, pi, (int)nblk, batch, out, out_stride_row, seed);
    return hipGetLastError();
}
