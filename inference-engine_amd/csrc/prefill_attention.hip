// Causal chunked-prefill attention over the int8 cache prefix, bf16 MFMA (gfx950).
//
// Semantics (qwen3-1.7b/kernels.py:987-1126 fed by dequantize_kv_prefix, kernels.py:868-932):
// packed row m of entry e attends to e's cached prefix — cache row slot_ids[e], columns
// [0, P), P = cu_cached[e+1] - cu_cached[e], k = q_int8 * k_scale * cal, v = q_int8 * v_scale —
// and to its own chunk rows [cu_seqlens[e], m] (bf16 k, v as given). Scores are
// dot(q, k) * D^-0.5 * log2(e); softmax in base 2; P is rounded to bf16 before PV;
// out = acc / l, or 0 when l == 0.
//
// Dequantization with the scales folded out of the tiles: int8 -> bf16 is exact, so the
// staged prefix tiles hold the raw integers and the scales go where they cost one multiply:
//   S(row, key) = (sum_d bf16(q[d] * cal[d]) * k_int8[key][d]) * (k_scale[key] * D^-0.5 log2 e)
//   PV          = sum_key bf16(p[key] * v_scale[key]) * v_int8[key][d]
// (the reference rounds bf16((k_int8 * k_scale) * cal) and bf16(v_int8 * v_scale) instead: same
// quantities, roundings in different places, well inside bf16 attention tolerance).
//
// Work: sub-blocks of up to 64 packed rows of one tile of `block_m` rows (tile_start, -1 = no
// work), both query heads of one KV head per workgroup. A sub-block's key range (prefix then
// chunk rows up to its last row) is cut into at most PF_MAXP pieces of >= PF_MIN_PIECE_TILES
// 64-key tiles; workgroup (sub-block * PF_MAXP + piece, kv head) takes one piece. Single-piece
// sub-blocks write `out` directly; the others write fp32 partials (acc, m, l) that
// prefill_combine_kernel merges (log-sum-exp). The grid depends on shapes only.
//
// Per 64-key tile: the workgroup stages K as [key][d] and V transposed as [d][key] in LDS, and
// the tile's score/probability scales; wave w (query head 2hk + (w & 1), rows 32 (w >> 1)..+32)
// computes
//   S^T (64 keys x 32 rows) = K . Q^T   v_mfma_f32_16x16x32_bf16, A = K from LDS, B = Q^T in VGPRs
//   online softmax on S^T (a lane holds one row's scores for 16 keys)
//   O^T (128 d x 32 rows) += V^T . P^T  A = V^T from LDS, B = P^T straight from the S^T
//                                       accumulators (same key permutation in A and B).
// The next tile's global loads are issued before the current tile's MFMA work.
#include "ie_common.h"

namespace ie {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int PF_BM = 64;  // packed rows per sub-block
constexpr int PF_BN = 64;  // keys per tile
constexpr int PF_D = 128;
constexpr int PF_THREADS = 256;
constexpr int PF_MAXP = 4;             // key pieces per sub-block, at most
constexpr int PF_MIN_PIECE_TILES = 4;  // tiles per piece, at least (when split)
constexpr float RESCALE_SLACK = 8.0f;  // log2 units

// LDS layouts (bytes), padded so that every fragment address is a per-lane base plus an
// immediate and the accesses are bank-conflict-free:
//   K tile: row = key, 256 B + 16 B pad; 16-byte unit c (8 channels) at c * 16.
//   V^T tile: row = channel d, 128 B (64 keys) + 16 B pad. Keys are stored in the order the PV
//   MFMA consumes them: within each 32-key half, position 8g + j holds key 4g + j (j < 4) and
//   key 16 + 4g + (j - 4) (j >= 4), so a lane's 8 keys for one 32-key step are one 16-byte read.
constexpr int KS_STRIDE = 272;
constexpr int VT_STRIDE = 144;
__device__ __forceinline__ int ks_off(int key, int c) { return key * KS_STRIDE + (c << 4); }
// byte offset of keys [4kg, 4kg + 4) of channel d
__device__ __forceinline__ int vt_off4(int d, int kg) {
    const int half = kg >> 3, k16 = kg & 7;  // kg: group of 4 keys within the 64-key tile
    const int pos = 32 * half + ((k16 & 3) << 3) + ((k16 >> 2) << 2);
    return d * VT_STRIDE + pos * 2;
}

// Sign-extended byte j of w as float (one v_cvt_f32_i32 with an SDWA byte select).
__device__ __forceinline__ float sbyte(uint32_t w, int j) {
    return (float)((int32_t)(w << (24 - 8 * j)) >> 24);
}
// bf16 pair from two floats whose low 16 bits are zero (exact small integers).
__device__ __forceinline__ uint32_t hi16pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

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
    float* part_acc;  // [N, Hq, PF_MAXP, 128]
    float* part_ml;   // [N, Hq, PF_MAXP, 2]
    int block_m, sub_per_tile, hq;
    float qk_scale;  // D^-0.5 * log2(e)
};

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

struct SubBlock {
    int r0, r1, seq_start, P, slot, npt, nct, ntiles, npieces;
};

// Rows and keys of sub-block `sb` (tile sb / sub_per_tile); false if it has no rows. Its keys
// are npt prefix tiles covering [0, P) and then nct chunk tiles covering chunk rows
// [seq_start, r1); a tile never mixes the two.
__device__ __forceinline__ bool sub_block(const PrefillArgs& a, int sb, SubBlock& s) {
    const int tile = sb / a.sub_per_tile, sub = sb - tile * a.sub_per_tile;
    const int row_start = uni(a.tile_start[tile]);
    if (row_start < 0) return false;
    const int seq = uni(a.seq_ids[row_start]);
    s.seq_start = uni(a.cu_seqlens[seq]);
    const int seq_end = uni(a.cu_seqlens[seq + 1]);
    s.r0 = row_start + sub * PF_BM;
    s.r1 = min(min(s.r0 + PF_BM, row_start + a.block_m), seq_end);
    if (s.r0 >= s.r1) return false;
    s.P = uni(a.cu_cached[seq + 1] - a.cu_cached[seq]);
    s.slot = uni(a.slot_ids[seq]);
    s.npt = (s.P + PF_BN - 1) / PF_BN;
    s.nct = (s.r1 - s.seq_start + PF_BN - 1) / PF_BN;
    s.ntiles = s.npt + s.nct;
    s.npieces = min(PF_MAXP, max(1, s.ntiles / PF_MIN_PIECE_TILES));
    return true;
}

// Global data of one tile, held in registers between its load and its LDS staging.
struct TileRegs {
    uint32_t kw[16];    // K: key tid>>2, channels [32 (tid&3), +32): int8 (8 words) or bf16
    uint32_t vw[4][4];  // V: keys 4 (tid&15) + u, channels [8 (tid>>4), +8): int8 (2) or bf16 (4)
    float kscale, kbias, vscale;  // prefix tiles, key tid (threads < 64): score scale, score
                                  // bias (-inf past P), P scale
};

// Buffer descriptors of one (sub-block, kv head): prefix K/V rows (128 B each, P rows) and scales
// of the cache, and the chunk's bf16 K/V rows [seq_start, r1). Reads past those ranges return 0.
struct TileSrc {
    rsrc_t pk, pv, pks, pvs, ck, cv;
    int ck_stride, cv_stride;  // bytes between chunk rows
};

__device__ __forceinline__ u32x4 ld128(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 ld64(rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ float ldf(rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Issue the loads of a tile. PREFIX: cache keys [kbase, kbase + 64) (int8; zeros at or past P).
// Otherwise chunk keys: packed rows seq_start + [kbase, kbase + 64) (bf16; zeros at or past the
// sub-block's last row). No branches: the buffer ranges do the masking.
template <bool PREFIX>
__device__ __forceinline__ void load_tile(TileRegs& r, const TileSrc& src, int kbase, int P,
                                          float qk_scale) {
    const int tid = threadIdx.x;
    {
        const int kk = kbase + (tid >> 2), q4 = tid & 3;
        if (PREFIX) {
            const int off = kk * PF_D + 32 * q4;
            const u32x4 b0 = ld128(src.pk, off), b1 = ld128(src.pk, off + 16);
            r.kw[0] = b0.x; r.kw[1] = b0.y; r.kw[2] = b0.z; r.kw[3] = b0.w;
            r.kw[4] = b1.x; r.kw[5] = b1.y; r.kw[6] = b1.z; r.kw[7] = b1.w;
        } else {
            const int off = kk * src.ck_stride + 64 * q4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 x = ld128(src.ck, off + 16 * i);
                r.kw[4 * i] = x.x; r.kw[4 * i + 1] = x.y; r.kw[4 * i + 2] = x.z; r.kw[4 * i + 3] = x.w;
            }
        }
    }
    {
        const int kg = tid & 15, dg = tid >> 4;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kk = kbase + 4 * kg + u;
            if (PREFIX) {
                const u32x2 b = ld64(src.pv, kk * PF_D + 8 * dg);
                r.vw[u][0] = b.x; r.vw[u][1] = b.y; r.vw[u][2] = 0u; r.vw[u][3] = 0u;
            } else {
                const u32x4 x = ld128(src.cv, kk * src.cv_stride + 16 * dg);
                r.vw[u][0] = x.x; r.vw[u][1] = x.y; r.vw[u][2] = x.z; r.vw[u][3] = x.w;
            }
        }
    }
    if (PREFIX && tid < PF_BN) {  // wave 0
        const int kk = kbase + tid;
        r.kscale = ldf(src.pks, 4 * kk) * qk_scale;
        r.kbias = kk < P ? 0.f : -INFINITY;
        r.vscale = ldf(src.pvs, 4 * kk);
    }
}

// Write a loaded tile to LDS: K as [key][d] bf16, V as [d][key] bf16 (int8 keys converted
// exactly), and for prefix tiles the per-key scales.
template <bool PREFIX>
__device__ __forceinline__ void stage_tile(const TileRegs& r, uint8_t* s_k, uint8_t* s_vt,
                                           float* s_ksc, float* s_kb, float* s_vsc) {
    const int tid = threadIdx.x;
    {
        const int key = tid >> 2, q4 = tid & 3;
        uint32_t w[16];
        if (PREFIX) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                w[2 * i] = hi16pair(sbyte(r.kw[i], 0), sbyte(r.kw[i], 1));
                w[2 * i + 1] = hi16pair(sbyte(r.kw[i], 2), sbyte(r.kw[i], 3));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i] = r.kw[i];
        }
        uint8_t* dst = s_k + ks_off(key, 4 * q4);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(dst + 16 * i) = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
    }
    {
        const int kg = tid & 15, dg = tid >> 4;
        uint8_t* dst = s_vt + vt_off4(8 * dg, kg);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t p01, p23;
            if (PREFIX) {  // channel j of key u: byte j of the key's 8 bytes
                p01 = hi16pair(sbyte(r.vw[0][j >> 2], j & 3), sbyte(r.vw[1][j >> 2], j & 3));
                p23 = hi16pair(sbyte(r.vw[2][j >> 2], j & 3), sbyte(r.vw[3][j >> 2], j & 3));
            } else {  // channel j of key u: bf16 half (j & 1) of word j >> 1
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                p01 = __builtin_amdgcn_perm(r.vw[1][j >> 1], r.vw[0][j >> 1], sel);
                p23 = __builtin_amdgcn_perm(r.vw[3][j >> 1], r.vw[2][j >> 1], sel);
            }
            *reinterpret_cast<u32x2*>(dst + j * VT_STRIDE) = u32x2{p01, p23};
        }
    }
    if (PREFIX && tid < PF_BN) {
        s_ksc[tid] = r.kscale;
        s_kb[tid] = r.kbias;
        s_vsc[tid] = r.vscale;
    }
}

// Per-wave running state: O^T accumulators (lane: d = 16mt + 4g + i, row = 16nt + l16) and the
// base-2 running max / sum of the lane's two rows.
struct WaveState {
    f32x4 acc[8][2];
    float m[2], l[2];
};

// MFMA + softmax work of one staged 64-key tile for one wave. PREFIX tiles: scores scaled per
// key, P scaled per key, keys past P masked (their scale is 0 and they are set to -inf).
// Chunk tiles: scores scaled by qk_scale, causal mask (chunk key c visible to row m iff
// seq_start + c <= m) and the range mask c < r1 - seq_start.
template <bool PREFIX>
__device__ __forceinline__ void tile_compute(WaveState& w, const bf16x8 (&qf)[2][4],
                                             const uint8_t* s_k, const uint8_t* s_vt,
                                             const float* s_ksc, const float* s_kb,
                                             const float* s_vsc, int kbase, int lim0, int lim1,
                                             float qk_scale, int l16, int g) {
    // ---- S^T = K . Q^T (64 keys x 32 rows) ----
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 st[4][2];
    const uint8_t* kfrag = s_k + ks_off(l16, g);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        __builtin_amdgcn_sched_barrier(0);  // bound live fragment registers per step
        bf16x8 kf[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            kf[ks] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(kfrag + 16 * mt * KS_STRIDE + 64 * ks));
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0], qf[nt][0], zero4, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < 4; ++ks)
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[nt][ks], c, 0, 0, 0);
            st[mt][nt] = c;
        }
    }
    // ---- scale, mask, online softmax (base 2) ----
    uint32_t pfrag[2][2][4];  // [32-key step][row tile] bf16x8 as 4 words
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        __builtin_amdgcn_sched_barrier(0);
        const int lim = nt ? lim1 : lim0;  // chunk tiles: last visible key index of this row
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 ksv = {qk_scale, qk_scale, qk_scale, qk_scale}, kbv = {0.f, 0.f, 0.f, 0.f};
            if (PREFIX) {
                ksv = *reinterpret_cast<const f32x4*>(s_ksc + 16 * mt + 4 * g);
                kbv = *reinterpret_cast<const f32x4*>(s_kb + 16 * mt + 4 * g);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x;
                if (PREFIX) {
                    x = __builtin_fmaf(st[mt][nt][i], ksv[i], kbv[i]);  // -inf past P
                } else {
                    const int kk = kbase + 16 * mt + 4 * g + i;
                    x = kk <= lim ? st[mt][nt][i] * ksv[i] : -INFINITY;
                }
                st[mt][nt][i] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        // Lazy max: the running max only moves when the tile's max exceeds it by more than
        // 2^RESCALE_SLACK, so probabilities stay <= 2^8 and the accumulators are rescaled rarely.
        const float mold = w.m[nt];
        const float mnew = mx > mold + RESCALE_SLACK ? mx : mold;
        const float msafe = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = __builtin_amdgcn_exp2f(mold - msafe);  // 1 if unchanged, 0 from -inf
        w.m[nt] = mnew;
        float lsum = 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 vsv = {1.f, 1.f, 1.f, 1.f};
            if (PREFIX) vsv = *reinterpret_cast<const f32x4*>(s_vsc + 16 * mt + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(st[mt][nt][i] - msafe);
                const float p1 = __builtin_amdgcn_exp2f(st[mt][nt][i + 1] - msafe);
                lsum += p0 + p1;
                pfrag[mt >> 1][nt][(mt & 1) * 2 + i / 2] =
                    PREFIX ? pack_bf16x2(p0 * vsv[i], p1 * vsv[i + 1]) : pack_bf16x2(p0, p1);
            }
        }
        w.l[nt] = w.l[nt] * alpha + lsum;
        if (__ballot(mnew != mold && mold != -INFINITY)) {  // accumulators are 0 before any key
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) w.acc[mt][nt] *= alpha;
        }
    }
    // ---- O^T += V^T . P^T ----
    const uint8_t* vfrag = s_vt + l16 * VT_STRIDE + 16 * g;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const bf16x8 vf = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(vfrag + 16 * mt * VT_STRIDE + 64 * s2));
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const bf16x8 pfv = __builtin_bit_cast(
                    bf16x8, u32x4{pfrag[s2][nt][0], pfrag[s2][nt][1], pfrag[s2][nt][2],
                                  pfrag[s2][nt][3]});
                w.acc[mt][nt] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pfv, w.acc[mt][nt], 0, 0, 0);
            }
        }
    }
}

// Q^T fragments of this wave: lane holds q[row = wr0 + 16nt + l16][d = 32ks + 8g .. +7], as
// bf16(q * cal) for prefix tiles or bf16 q for chunk tiles; zero rows past the sub-block.
template <bool PREFIX>
__device__ __forceinline__ void load_q(bf16x8 (&qf)[2][4], const PrefillArgs& a, int wr0, int r1,
                                       int h, const float* cal, int l16, int g) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int row = wr0 + 16 * nt + l16;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 w = {0u, 0u, 0u, 0u};
            if (row < r1)
                w = *reinterpret_cast<const u32x4*>(a.q + row * a.q_st + h * a.q_sh + 32 * ks + 8 * g);
            if (PREFIX) {
                const f32x4 c0 = *reinterpret_cast<const f32x4*>(cal + 32 * ks + 8 * g);
                const f32x4 c1 = *reinterpret_cast<const f32x4*>(cal + 32 * ks + 8 * g + 4);
                w = u32x4{pack_bf16x2(bf16lo(w.x) * c0[0], bf16hi(w.x) * c0[1]),
                          pack_bf16x2(bf16lo(w.y) * c0[2], bf16hi(w.y) * c0[3]),
                          pack_bf16x2(bf16lo(w.z) * c1[0], bf16hi(w.z) * c1[1]),
                          pack_bf16x2(bf16lo(w.w) * c1[2], bf16hi(w.w) * c1[3])};
            }
            qf[nt][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }
}

#ifndef IE_PREFILL_WG_PER_CU
#define IE_PREFILL_WG_PER_CU 2
#endif

__global__ __launch_bounds__(PF_THREADS, IE_PREFILL_WG_PER_CU) void prefill_attention_kernel(
    PrefillArgs a) {
    const int sb = blockIdx.x / PF_MAXP, piece = blockIdx.x % PF_MAXP;
    const int hk = blockIdx.y;
    SubBlock s;
    if (!sub_block(a, sb, s) || piece >= s.npieces) return;
    const int kt_begin = piece * s.ntiles / s.npieces;
    const int kt_end = (piece + 1) * s.ntiles / s.npieces;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int h = 2 * hk + (wave & 1);
    const int wr0 = s.r0 + 32 * (wave >> 1);  // first row of this wave

    // two tile buffers: tile i is staged into buffer i & 1 while the other one is computed on
    __shared__ __attribute__((aligned(16))) uint8_t s_k[2][PF_BN * KS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint8_t s_vt[2][PF_D * VT_STRIDE];
    __shared__ __attribute__((aligned(16))) float s_ksc[2][PF_BN];
    __shared__ __attribute__((aligned(16))) float s_kb[2][PF_BN];
    __shared__ __attribute__((aligned(16))) float s_vsc[2][PF_BN];

    const float* cal = a.c.k_calibration + s.slot * a.c.cal_stride_slot + hk * a.c.cal_stride_head;
    TileSrc src;
    {
        const int64_t crow = s.slot * a.c.stride_slot + hk * a.c.stride_head;
        const int64_t srow = s.slot * a.c.scale_stride_slot + hk * a.c.scale_stride_head;
        src.pk = make_rsrc(a.c.k + crow, (uint32_t)s.P * PF_D);
        src.pv = make_rsrc(a.c.v + crow, (uint32_t)s.P * PF_D);
        src.pks = make_rsrc(a.c.k_scale + srow, (uint32_t)s.P * 4);
        src.pvs = make_rsrc(a.c.v_scale + srow, (uint32_t)s.P * 4);
        const int nrows = s.r1 - s.seq_start;  // chunk rows visible to this sub-block
        src.ck_stride = (int)a.k_st * 2;
        src.cv_stride = (int)a.v_st * 2;
        src.ck = make_rsrc(a.k + s.seq_start * a.k_st + hk * a.k_sh, (uint32_t)(nrows * src.ck_stride));
        src.cv = make_rsrc(a.v + s.seq_start * a.v_st + hk * a.v_sh, (uint32_t)(nrows * src.cv_stride));
    }

    // chunk tiles: last visible chunk key of each of this lane's two rows
    const int rowA = wr0 + l16, rowB = wr0 + 16 + l16;
    const int clim = s.r1 - s.seq_start - 1;
    const int lim0 = min(rowA - s.seq_start, clim), lim1 = min(rowB - s.seq_start, clim);

    // tile kt: prefix tile kt (keys [64kt, ..)) if kt < npt, else chunk tile kt - npt
    auto load = [&](TileRegs& r, int kt) {
        if (kt < s.npt) load_tile<true>(r, src, kt * PF_BN, s.P, a.qk_scale);
        else load_tile<false>(r, src, (kt - s.npt) * PF_BN, s.P, a.qk_scale);
    };
    auto stage = [&](const TileRegs& r, int kt, int buf) {
        if (kt < s.npt) stage_tile<true>(r, s_k[buf], s_vt[buf], s_ksc[buf], s_kb[buf], s_vsc[buf]);
        else stage_tile<false>(r, s_k[buf], s_vt[buf], s_ksc[buf], s_kb[buf], s_vsc[buf]);
    };

    WaveState ws;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) ws.acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    ws.m[0] = ws.m[1] = -INFINITY;
    ws.l[0] = ws.l[1] = 0.f;

    TileRegs pf;
    load(pf, kt_begin);
    stage(pf, kt_begin, 0);
    bf16x8 qf[2][4];
    int kt = kt_begin;
    const int prefix_end = min(kt_end, s.npt);
    if (kt < prefix_end) {
        load_q<true>(qf, a, wr0, s.r1, h, cal, l16, g);
        __syncthreads();
        for (; kt < prefix_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            const bool has_next = kt + 1 < kt_end;
            if (has_next) load(pf, kt + 1);  // in flight during this tile's MFMA work
            tile_compute<true>(ws, qf, s_k[buf], s_vt[buf], s_ksc[buf], s_kb[buf], s_vsc[buf],
                               kt * PF_BN, 0, 0, a.qk_scale, l16, g);
            if (has_next) stage(pf, kt + 1, buf ^ 1);
            __syncthreads();  // next buffer staged; this buffer free for tile kt + 2
        }
    }
    if (kt < kt_end) {
        load_q<false>(qf, a, wr0, s.r1, h, cal, l16, g);
        if (kt == kt_begin) __syncthreads();
        for (; kt < kt_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            const bool has_next = kt + 1 < kt_end;
            const int kc = (kt - s.npt) * PF_BN;
            if (has_next) load_tile<false>(pf, src, kc + PF_BN, s.P, a.qk_scale);
            tile_compute<false>(ws, qf, s_k[buf], s_vt[buf], s_ksc[buf], s_kb[buf], s_vsc[buf],
                                kc, lim0, lim1, a.qk_scale, l16, g);
            if (has_next) stage_tile<false>(pf, s_k[buf ^ 1], s_vt[buf ^ 1], s_ksc[buf ^ 1],
                                            s_kb[buf ^ 1], s_vsc[buf ^ 1]);
            __syncthreads();
        }
    }

    // ---- results: lane holds row = wr0 + 16nt + l16, channels d = 16mt + 4g + i ----
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float l = ws.l[nt];
        l += shfl_xor(l, 16);
        l += shfl_xor(l, 32);
        const int row = wr0 + 16 * nt + l16;
        if (row >= s.r1) continue;
        if (s.npieces == 1) {
            uint16_t* o = a.out + row * a.o_st + h * a.o_sh;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                const f32x4 x = ws.acc[mt][nt];
                float y[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = l != 0.f ? x[i] / l : 0.f;
                *reinterpret_cast<u32x2*>(o + 16 * mt + 4 * g) =
                    u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
            }
        } else {
            const int64_t prow = ((int64_t)row * a.hq + h) * PF_MAXP + piece;
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
                *reinterpret_cast<f32x4*>(a.part_acc + prow * PF_D + 16 * mt + 4 * g) = ws.acc[mt][nt];
            if (g == 0)
                *reinterpret_cast<float2*>(a.part_ml + prow * 2) = make_float2(ws.m[nt], l);
        }
    }
}

constexpr int PF_COMB_SPLIT = 16;  // combine workgroups per sub-block (8 (row, head) pairs each)

// grid (num_tiles * sub_per_tile * PF_COMB_SPLIT, Hkv), block 256: merges the pieces of split
// sub-blocks (log-sum-exp, base 2). 32 threads per (row, query head), 4 channels each; every
// thread issues all of its loads up front.
__global__ __launch_bounds__(PF_THREADS) void prefill_combine_kernel(PrefillArgs a) {
    const int hk = blockIdx.y;
    SubBlock s;
    if (!sub_block(a, blockIdx.x / PF_COMB_SPLIT, s) || s.npieces <= 1) return;
    const int tid = threadIdx.x;
    const int pair = (blockIdx.x % PF_COMB_SPLIT) * 8 + (tid >> 5);  // 0..127
    const int row = s.r0 + (pair >> 1);
    if (row >= s.r1) return;
    const int h = 2 * hk + (pair & 1);
    const int d = 4 * (tid & 31);
    const int64_t prow = ((int64_t)row * a.hq + h) * PF_MAXP;
    float2 ml[PF_MAXP];
    f32x4 acc[PF_MAXP];
#pragma unroll
    for (int p = 0; p < PF_MAXP; ++p) {
        ml[p] = make_float2(-INFINITY, 0.f);
        acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (p < s.npieces) {
            ml[p] = *reinterpret_cast<const float2*>(a.part_ml + (prow + p) * 2);
            acc[p] = *reinterpret_cast<const f32x4*>(a.part_acc + (prow + p) * PF_D + d);
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int p = 0; p < PF_MAXP; ++p) mx = fmaxf(mx, ml[p].x);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int p = 0; p < PF_MAXP; ++p) {
        const float w = ml[p].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[p].x - mx);
        num += acc[p] * w;
        den += ml[p].y * w;
    }
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = den != 0.f ? num[i] / den : 0.f;
    *reinterpret_cast<u32x2*>(a.out + row * a.o_st + h * a.o_sh + d) =
        u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
}

static size_t prefill_workspace_bytes(int64_t num_tokens, int hq) {
    return (size_t)num_tokens * hq * PF_MAXP * (PF_D + 2) * sizeof(float);
}

}  // namespace ie

using namespace ie;

extern "C" size_t ie_prefill_attention_workspace_size(int64_t num_tokens, int32_t num_q_heads) {
    return prefill_workspace_bytes(std::max<int64_t>(num_tokens, 0), std::max(num_q_heads, 0));
}

extern "C" hipError_t ie_prefill_attention(
    const ie_bf16* q, int64_t q_stride_tok, int64_t q_stride_head, const ie_bf16* k,
    int64_t k_stride_tok, int64_t k_stride_head, const ie_bf16* v, int64_t v_stride_tok,
    int64_t v_stride_head, int64_t num_tokens, int32_t num_q_heads, const int32_t* seq_ids,
    const int32_t* cu_seqlens, const int32_t* tile_start, int32_t num_tiles, int32_t block_m,
    const ie_kv_cache* cache, const int32_t* slot_ids, const int32_t* cu_cached, ie_bf16* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
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
    // chunk rows are read through 32-bit buffer ranges whose end masks rows past the sub-block
    IE_REQUIRE(k_stride_tok >= PF_D && v_stride_tok >= PF_D,
               "k/v token stride must be at least head_dim elements");
    IE_REQUIRE(num_tokens * std::max(k_stride_tok, v_stride_tok) * 2 < ((int64_t)1 << 31),
               "k/v too large for 32-bit row offsets");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(cache->k_calibration) & 15) == 0 &&
                   cache->cal_stride_head % 4 == 0 && cache->cal_stride_slot % 4 == 0,
               "k_calibration rows must be 16-byte aligned");
    const size_t need = prefill_workspace_bytes(num_tokens, num_q_heads);
    IE_REQUIRE(workspace != nullptr && workspace_bytes >= need && al16(workspace),
               "workspace too small");
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
    a.part_acc = (float*)workspace;
    a.part_ml = a.part_acc + (size_t)num_tokens * num_q_heads * PF_MAXP * PF_D;
    a.block_m = block_m;
    a.sub_per_tile = (block_m + PF_BM - 1) / PF_BM;
    a.hq = num_q_heads;
    a.qk_scale = (float)(0.08838834764831845 * 1.4426950408889634);  // D^-0.5 * log2(e), D = 128
    const unsigned nsb = (unsigned)num_tiles * a.sub_per_tile;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(nsb * PF_MAXP, cache->num_kv_heads),
                       dim3(PF_THREADS), 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prefill_combine_kernel, dim3(nsb * PF_COMB_SPLIT, cache->num_kv_heads),
                       dim3(PF_THREADS), 0, stream, a);
    return hipGetLastError();
}
