// y[M, N] = x[M, K] . W[N, K]^T for few rows (decode, M <= 64), bf16 in, fp32 accumulation, bf16 out
// (gfx950). Replaces qwen3-1.7b/kernels.py:1373-1443 `skinny_matmul` (the `linear` of
// kernels.py:1451-1458 picks it or the library per shape).
//
// At decode row counts the weight read is the whole cost (one byte of W feeds 2M flops), so the
// kernel streams every weight byte once from HBM and keeps x, which every workgroup needs, in the
// caches. Workgroup n-tile t (grid N / 16, 512 threads) owns W rows [16t, 16t + 16); its eight
// waves split K into eight contiguous slices. Per 32-wide k step a wave issues
// v_mfma_f32_16x16x32_bf16 with A = 16 W rows x 32 k (lane (r, g) holds row 16t + r, k 8g..8g+7:
// one 16-byte load) and B = x^T, 32 k x 16 rows of x per m-tile (the same lane mapping over x's
// rows), so D = y^T (16 n x 16 m). Loads run SG_UNROLL steps ahead of the MFMAs. The eight
// partial D tiles are summed through LDS in wave order and written as bf16.
#include "ie_common.h"

namespace ie {

typedef __bf16 sg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sg_f32x4 __attribute__((ext_vector_type(4)));

constexpr int SG_WAVES = 8;
constexpr int SG_THREADS = SG_WAVES * IE_WAVE;
constexpr int SG_UNROLL = 4;  // k steps of 32 in flight per wave

__device__ __forceinline__ sg_bf16x8 ld_frag(rsrc_t r, int off) {
    return __builtin_bit_cast(sg_bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// MT m-tiles of 16 rows (M <= 16 MT), NT n-tiles of 16 weight rows per workgroup (every x
// fragment feeds NT MFMAs). K a multiple of 8 * 32 = 256 (each wave's slice is a multiple of 32).
template <int MT, int NT>
__global__ __launch_bounds__(SG_THREADS) void skinny_gemm_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, const uint16_t* __restrict__ w, int64_t ws,
    int K, uint16_t* __restrict__ y, int64_t ys) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * NT;
    // wave w of workgroup b takes K slice (w + b) mod 8: neighbouring workgroups read different
    // parts of x at any moment instead of all hitting the same L2 lines
    const int kw = K / SG_WAVES, k_begin = (int)((wave + blockIdx.x) % SG_WAVES) * kw;
    // W rows [n0, n0 + 16 NT) and x rows [0, M): the buffer ranges zero the rows of x past M
    const rsrc_t rw = make_rsrc(w + (int64_t)n0 * ws, (uint32_t)(16 * NT * ws * 2));
    const rsrc_t rx = make_rsrc(x, (uint32_t)(M * xs * 2));
    int woff[NT], xoff[MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) woff[nt] = ((16 * nt + l16) * (int)ws + k_begin + 8 * g) * 2;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xoff[mt] = ((16 * mt + l16) * (int)xs + k_begin + 8 * g) * 2;

    sg_f32x4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = sg_f32x4{0.f, 0.f, 0.f, 0.f};
    const int steps = kw / 32;
    for (int s = 0; s < steps; s += SG_UNROLL) {
        sg_bf16x8 wf[SG_UNROLL][NT], xf[SG_UNROLL][MT];
#pragma unroll
        for (int u = 0; u < SG_UNROLL; ++u) {
            const int o = (s + u < steps ? s + u : steps) * 64;  // past the slice: out of range
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) wf[u][nt] = ld_frag(rw, s + u < steps ? woff[nt] + o : -1);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) xf[u][mt] = ld_frag(rx, s + u < steps ? xoff[mt] + o : -1);
        }
#pragma unroll
        for (int u = 0; u < SG_UNROLL; ++u)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[u][nt], xf[u][mt],
                                                                         acc[nt][mt], 0, 0, 0);
    }

    // D lane (l16, g) element i: n = n0 + 16 nt + 4g + i, m = 16 mt + l16. The waves' partial
    // tiles are summed in wave order, one (nt, mt) tile per wave.
    __shared__ sg_f32x4 s_acc[SG_WAVES][NT * MT][IE_WAVE];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) s_acc[wave][nt * MT + mt][lane] = acc[nt][mt];
    __syncthreads();
    for (int tile = wave; tile < NT * MT; tile += SG_WAVES) {
        sg_f32x4 t = s_acc[0][tile][lane];
#pragma unroll
        for (int v = 1; v < SG_WAVES; ++v) t += s_acc[v][tile][lane];
        const int nt = tile / MT, mt = tile % MT;
        const int m = 16 * mt + l16;
        if (m < M) {
            uint16_t* dst = y + (int64_t)m * ys + n0 + 16 * nt + 4 * g;
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(pack_bf16x2(t[0], t[1]), pack_bf16x2(t[2], t[3]));
        }
    }
}

}  // namespace ie

using namespace ie;

extern "C" hipError_t ie_skinny_gemm(const ie_bf16* x, int64_t x_stride, int32_t m,
                                     const ie_bf16* weight, int64_t weight_stride, int32_t n,
                                     int32_t k, int32_t n_tiles, ie_bf16* y, int64_t y_stride,
                                     hipStream_t stream) {
    IE_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative sizes");
    if (m == 0 || n == 0) return hipSuccess;
    IE_REQUIRE(x && weight && y, "null pointer");
    IE_REQUIRE(m <= 64, "at most 64 rows");
    IE_REQUIRE(n % 16 == 0 && k % (SG_WAVES * 32) == 0 && k > 0,
               "n must be a multiple of 16 and k of 256");
    IE_REQUIRE(n_tiles == 1 || n_tiles == 2 || n_tiles == 4, "n_tiles must be 1, 2 or 4");
    IE_REQUIRE(n % (16 * n_tiles) == 0, "n must be a multiple of 16 n_tiles");
    IE_REQUIRE(x_stride % 8 == 0 && weight_stride % 8 == 0 && y_stride % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 7) == 0,
               "rows must be 16-byte aligned (8-byte for y)");
    IE_REQUIRE((int64_t)m * x_stride * 2 < (1LL << 31) &&
                   16LL * n_tiles * weight_stride * 2 < (1LL << 31),
               "operands too large for 32-bit buffer offsets");
    const dim3 grid((unsigned)(n / (16 * n_tiles)));
    const int mt = (m + 15) / 16;
#define IE_SG_LAUNCH(MT, NT)                                                                   \
    hipLaunchKernelGGL((skinny_gemm_kernel<MT, NT>), grid, dim3(SG_THREADS), 0, stream,        \
                       (const uint16_t*)x, x_stride, m, (const uint16_t*)weight, weight_stride, \
                       k, (uint16_t*)y, y_stride)
#define IE_SG_NT(MT)                                 \
    switch (n_tiles) {                               \
        case 1: IE_SG_LAUNCH(MT, 1); break;          \
        case 2: IE_SG_LAUNCH(MT, 2); break;          \
        default: IE_SG_LAUNCH(MT, 4); break;         \
    }
    switch (mt) {
        case 1: IE_SG_NT(1); break;
        case 2: IE_SG_NT(2); break;
        case 3: IE_SG_NT(3); break;
        default: IE_SG_NT(4); break;
    }
#undef IE_SG_NT
#undef IE_SG_LAUNCH
    return hipGetLastError();
}
