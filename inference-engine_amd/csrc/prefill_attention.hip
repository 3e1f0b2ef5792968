// Causal chunked-prefill attention over the int8 cache prefix, bf16 MFMA (gfx950).
//
// Semantics (qwen3-1.7b/kernels.py:987-1126 fed by dequantize_kv_prefix, kernels.py:868-932):
// packed row m of entry e attends to e's cached prefix — cache row slot_ids[e], columns
// [0, P), P = cu_cached[e+1] - cu_cached[e], dequantized as k = bf16((q * k_scale) * cal),
// v = bf16(q * v_scale) — and to its own chunk rows [cu_seqlens[e], m] (bf16 k, v as given).
// Scores are dot(q, k) * D^-0.5 * log2(e); softmax in base 2; P is rounded to bf16 before PV;
// out = acc / l, or 0 when l == 0.
//
// Work: workgroup (x, kv head) takes sub-block x % SUB of tile x / SUB, i.e. up to 64 rows of
// one tile of `block_m` rows (tile_start, -1 = no work), for both query heads of the KV head.
// Wave w computes query head 2*hk + (w & 1) for rows 32*(w >> 1) .. +32 of the sub-block.
//
// Per 64-key tile: the workgroup stages K as [key][d] and V transposed as [d][key] in LDS
// (bf16; prefix keys dequantized on the way in), then each wave computes
//   S^T (64 keys x 32 rows) = K . Q^T   with v_mfma_f32_16x16x32_bf16 (A = K from LDS, B = Q^T
//                                        held in registers),
//   online softmax on S^T (a lane holds one row's scores for 16 keys), and
//   O^T (128 d x 32 rows) += V^T . P^T  (A = V^T from LDS, B = P^T straight from the S^T
//                                        accumulators: the key order inside a 32-key step is
//                                        permuted identically in A and B, so no shuffle).
#include "ie_common.h"

namespace ie {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int PF_BM = 64;   // packed rows per workgroup
constexpr int PF_BN = 64;   // keys per tile
constexpr int PF_D = 128;
constexpr int PF_THREADS = 256;
constexpr float LOG2E = 1.4426950408889634f;

// LDS layouts (bytes). K tile: row = key (256 B), 16-byte unit c of 8 channels stored at
// c ^ (key & 15). V^T tile: row = channel d (128 B), 8-byte unit u of 4 keys stored at
// u ^ ((d ^ (d >> 4)) & 15). Both swizzles keep the fragment reads and the staging writes free
// of bank conflicts.
__device__ __forceinline__ int ks_off(int key, int c) { return key * 256 + ((c ^ (key & 15)) << 4); }
__device__ __forceinline__ int vt_off(int d, int u) {
    return d * 128 + ((u ^ ((d ^ (d >> 4)) & 15)) << 3);
}

__device__ __forceinline__ uint32_t pack_rne(float lo, float hi) { return pack_bf16x2(lo, hi); }

struct PrefillArgs {
    const uint16_t* q;
    int64_t q_st, q_sh;
    const uint16_t* k;
    int64_t k_st, k_sh;
    const uint16_t* v;
    int64_t v_st, v_sh;
    const int32_t* seq_ids;
    const int32_t* cu_seqlens;
    const int32_t* tile_start;
    const int32_t* slot_ids;
    const int32_t* cu_cached;
    ie_kv_cache c;
    uint16_t* out;
    int64_t o_st, o_sh;
    int block_m, sub_per_tile, hq;
    float qk_scale;  // D^-0.5 * log2(e)
};

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

__global__ __launch_bounds__(PF_THREADS) void prefill_attention_kernel(PrefillArgs a) {
    const int tile = blockIdx.x / a.sub_per_tile;
    const int sub = blockIdx.x % a.sub_per_tile;
    const int hk = blockIdx.y;
    const int row_start = uni(a.tile_start[tile]);
    if (row_start < 0) return;
    const int seq = uni(a.seq_ids[row_start]);
    const int seq_start = uni(a.cu_seqlens[seq]);
    const int seq_end = uni(a.cu_seqlens[seq + 1]);
    const int r0 = row_start + sub * PF_BM;
    const int r1 = min(min(r0 + PF_BM, row_start + a.block_m), seq_end);
    if (r0 >= r1) return;
    const int P = uni(a.cu_cached[seq + 1] - a.cu_cached[seq]);
    const int slot = uni(a.slot_ids[seq]);
    const int T = P + (r1 - seq_start);  // keys: prefix then chunk rows [seq_start, r1)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int h = 2 * hk + (wave & 1);
    const int wr0 = r0 + 32 * (wave >> 1);  // first row of this wave

    __shared__ __attribute__((aligned(16))) uint8_t s_k[PF_BN * 256];
    __shared__ __attribute__((aligned(16))) uint8_t s_vt[PF_D * 128];
    __shared__ float s_cal[PF_D];

    const float* calp = a.c.k_calibration + slot * a.c.cal_stride_slot + hk * a.c.cal_stride_head;
    if (tid < PF_D) s_cal[tid] = calp[tid];

    // ---- Q^T fragments: lane holds Q[row = wr0 + 16nt + l16][d = 32ks + 8g .. +7] ----
    bf16x8 qf[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int row = wr0 + 16 * nt + l16;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 w = {0u, 0u, 0u, 0u};
            if (row < r1)
                w = *reinterpret_cast<const u32x4*>(a.q + row * a.q_st + h * a.q_sh + 32 * ks + 8 * g);
            qf[nt][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }

    f32x4 acc[8][2];  // O^T: [d tile][row tile], lane holds d = 16mt + 4g + i, row = 16nt + l16
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

    const int8_t* kc = a.c.k + slot * a.c.stride_slot + hk * a.c.stride_head;
    const int8_t* vc = a.c.v + slot * a.c.stride_slot + hk * a.c.stride_head;
    const float* ksc = a.c.k_scale + slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;
    const float* vsc = a.c.v_scale + slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;

    const int n_tiles = (T + PF_BN - 1) / PF_BN;
    for (int kt = 0; kt < n_tiles; ++kt) {
        const int kbase = kt * PF_BN;
        __syncthreads();  // previous tile fully consumed (and s_cal visible on the first pass)
        // ---- stage K: thread -> key tid >> 2, channels [32q, 32q + 32) ----
        {
            const int key = tid >> 2, q4 = tid & 3;
            const int kk = kbase + key;
            uint32_t w[16];
            if (kk < P) {
                const u32x4 b0 = *reinterpret_cast<const u32x4*>(kc + (int64_t)kk * PF_D + 32 * q4);
                const u32x4 b1 = *reinterpret_cast<const u32x4*>(kc + (int64_t)kk * PF_D + 32 * q4 + 16);
                const float sk = ksc[kk];
                const uint32_t bytes[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        const int d = 32 * q4 + 4 * i + j;
                        const float x0 = (float)(int8_t)(bytes[i] >> (8 * j));
                        const float x1 = (float)(int8_t)(bytes[i] >> (8 * j + 8));
                        w[2 * i + j / 2] = pack_rne(__fmul_rn(__fmul_rn(x0, sk), s_cal[d]),
                                                    __fmul_rn(__fmul_rn(x1, sk), s_cal[d + 1]));
                    }
                }
            } else if (kk < T) {
                const uint16_t* src = a.k + (int64_t)(seq_start + kk - P) * a.k_st + hk * a.k_sh + 32 * q4;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const u32x4 x = *reinterpret_cast<const u32x4*>(src + 8 * i);
                    w[4 * i] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) w[i] = 0u;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<u32x4*>(s_k + ks_off(key, 4 * q4 + i)) =
                    u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
        }
        // ---- stage V^T: thread -> keys 4kg .. 4kg+3, channels [8dg, 8dg + 8) ----
        {
            const int kg = tid >> 4, dg = tid & 15;
            float vf[4][8];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int kk = kbase + 4 * kg + u;
                if (kk < P) {
                    const u32x2 b = *reinterpret_cast<const u32x2*>(vc + (int64_t)kk * PF_D + 8 * dg);
                    const float sv = vsc[kk];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t wd = j < 4 ? b.x : b.y;
                        vf[u][j] = __fmul_rn((float)(int8_t)(wd >> (8 * (j & 3))), sv);
                    }
                } else if (kk < T) {
                    const u32x4 x = *reinterpret_cast<const u32x4*>(
                        a.v + (int64_t)(seq_start + kk - P) * a.v_st + hk * a.v_sh + 8 * dg);
                    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        vf[u][2 * j] = bf16lo(xs[j]);
                        vf[u][2 * j + 1] = bf16hi(xs[j]);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) vf[u][j] = 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 8 * dg + j;
                *reinterpret_cast<u32x2*>(s_vt + vt_off(d, kg)) =
                    u32x2{pack_rne(vf[0][j], vf[1][j]), pack_rne(vf[2][j], vf[3][j])};
            }
        }
        __syncthreads();

        // ---- S^T = K . Q^T for 64 keys x 32 rows ----
        f32x4 st[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            bf16x8 kf[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                kf[ks] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(s_k + ks_off(16 * mt + l16, 4 * ks + g)));
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[nt][ks], c, 0, 0, 0);
                st[mt][nt] = c;
            }
        }
        // ---- mask, online softmax (base 2) ----
        uint32_t pfrag[2][2][4];  // [32-key step][row tile] bf16x8 as 4 dwords
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int row = wr0 + 16 * nt + l16;  // packed row of this lane's column
            float sv[4][4];
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int kk = kbase + 16 * mt + 4 * g + i;
                    float x = st[mt][nt][i] * a.qk_scale;
                    const bool ok = kk < P || (kk < T && seq_start + (kk - P) <= row);
                    x = ok ? x : -INFINITY;
                    sv[mt][i] = x;
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, shfl_xor(mx, 16));
            mx = fmaxf(mx, shfl_xor(mx, 32));
            const float mnew = fmaxf(m_run[nt], mx);
            const float msafe = mnew == -INFINITY ? 0.f : mnew;
            const float alpha = __builtin_amdgcn_exp2f(m_run[nt] - msafe);
            m_run[nt] = mnew;
            float lsum = 0.f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(sv[mt][i] - msafe);
                    const float p1 = __builtin_amdgcn_exp2f(sv[mt][i + 1] - msafe);
                    lsum += p0 + p1;
                    pfrag[mt >> 1][nt][(mt & 1) * 2 + i / 2] = pack_rne(p0, p1);
                }
            l_run[nt] = l_run[nt] * alpha + lsum;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) acc[mt][nt] *= alpha;
        }
        // ---- O^T += V^T . P^T ----
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const int d = 16 * mt + l16;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const u32x2 lo = *reinterpret_cast<const u32x2*>(s_vt + vt_off(d, 8 * s2 + g));
                const u32x2 hi = *reinterpret_cast<const u32x2*>(s_vt + vt_off(d, 8 * s2 + 4 + g));
                const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const bf16x8 pf = __builtin_bit_cast(
                        bf16x8, u32x4{pfrag[s2][nt][0], pfrag[s2][nt][1], pfrag[s2][nt][2],
                                      pfrag[s2][nt][3]});
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, acc[mt][nt], 0, 0, 0);
                }
            }
        }
    }

    // ---- normalise and store: lane holds out[row = wr0 + 16nt + l16][h][d = 16mt + 4g + i] ----
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float l = l_run[nt];
        l += shfl_xor(l, 16);
        l += shfl_xor(l, 32);
        const int row = wr0 + 16 * nt + l16;
        if (row >= r1) continue;
        const float inv = l != 0.f ? 1.0f / l : 0.f;
        uint16_t* o = a.out + row * a.o_st + h * a.o_sh;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {
            const f32x4 x = acc[mt][nt];
            const float y0 = l != 0.f ? x[0] / l : 0.f, y1 = l != 0.f ? x[1] / l : 0.f;
            const float y2 = l != 0.f ? x[2] / l : 0.f, y3 = l != 0.f ? x[3] / l : 0.f;
            (void)inv;
            *reinterpret_cast<u32x2*>(o + 16 * mt + 4 * g) = u32x2{pack_rne(y0, y1), pack_rne(y2, y3)};
        }
    }
}

}  // namespace ie

using namespace ie;

extern "C" hipError_t ie_prefill_attention(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, hipStream_t stream) {
    hipError_t e = check_cache(cache);
    if (e != hipSuccess) return e;
    IE_REQUIRE(num_tokens >= 0 && num_tiles >= 0, "negative sizes");
    IE_REQUIRE(block_m > 0, "block_m must be positive");
    IE_REQUIRE(num_q_heads == 2 * cache->num_kv_heads, "num_q_heads must be 2 * num_kv_heads");
    if (num_tokens == 0 || num_tiles == 0) return hipSuccess;
    IE_REQUIRE(q && k && v && seq_ids && cu_seqlens && tile_start && slot_ids && cu_cached && out,
               "null pointer");
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    IE_REQUIRE(al16(q) && al16(k) && al16(v) && al16(out), "q/k/v/out must be 16-byte aligned");
    IE_REQUIRE(q_stride_tok % 8 == 0 && q_stride_head % 8 == 0 && k_stride_tok % 8 == 0 &&
                   k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 && v_stride_head % 8 == 0 &&
                   out_stride_tok % 4 == 0 && out_stride_head % 4 == 0,
               "q/k/v/out rows must be 16-byte aligned with contiguous head_dim");
    PrefillArgs a;
    a.q = (const uint16_t*)q;
    a.q_st = q_stride_tok;
    a.q_sh = q_stride_head;
    a.k = (const uint16_t*)k;
    a.k_st = k_stride_tok;
    a.k_sh = k_stride_head;
    a.v = (const uint16_t*)v;
    a.v_st = v_stride_tok;
    a.v_sh = v_stride_head;
    a.seq_ids = seq_ids;
    a.cu_seqlens = cu_seqlens;
    a.tile_start = tile_start;
    a.slot_ids = slot_ids;
    a.cu_cached = cu_cached;
    a.c = *cache;
    a.out = (uint16_t*)out;
    a.o_st = out_stride_tok;
    a.o_sh = out_stride_head;
    a.block_m = block_m;
    a.sub_per_tile = (block_m + PF_BM - 1) / PF_BM;
    a.hq = num_q_heads;
    a.qk_scale = (float)(0.08838834764831845 * 1.4426950408889634);  // D^-0.5 * log2(e), D = 128
    dim3 grid((unsigned)num_tiles * a.sub_per_tile, (unsigned)cache->num_kv_heads);
    hipLaunchKernelGGL(prefill_attention_kernel, grid, dim3(PF_THREADS), 0, stream, a);
    return hipGetLastError();
}
